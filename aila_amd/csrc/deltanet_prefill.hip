// Gated DeltaNet chunked prefill on gfx950 (WY/UT form, chunk C = 64).
//
// Reference: Qwen35HybridTextBackend::run_linear_delta_prefill_gpu_batched
// (src/models/Qwen35HybridTextBackend.cpp:1306-1508) applies the decode
// recurrence token by token inside one workgroup per value head. Here the
// same recurrence (host form :1729-1780) is evaluated chunk-wise:
//
// For a chunk with state S0 [dk, dv] (rows = key dims), normalisers
// ik_t = 1/sqrt(|k_t|^2+eps), iq_t likewise, beta_t, cumulative log-decay
// G_t = sum_{s<=t} g_t, and the raw bf16 inputs K, Q, V (exact in bf16):
//   A[t,s]  = beta_t e^(G_t-G_s) ik_t ik_s (K K^T)[t,s]          (s < t)
//   T       = (I + A)^-1,  To = T - I                            (fp32)
//   W       = bf16(To diag(sw)) K + diag(sw) K,   sw = beta e^G ik
//   U       = bf16(To diag(beta)) V + diag(beta) V
//   D       = U - W S0
//   O       = scale * ( fq (Q S0) + P D ),   fq = e^G iq,
//             P[t,s] = e^(G_t-G_s) iq_t ik_s (Q K^T)[t,s]          (s <= t)
//   S1      = e^(G_last) S0 + K^T (fk D),      fk = e^(G_last-G) ik
// All decays are formed as exp of differences with s <= t (never a ratio),
// so they stay in [0, 1]. T is computed in fp32 (diagonal 16x16 blocks by
// substitution, off-diagonal blocks on the fp32 matrix cores), the diagonal
// of T is applied in fp32, and every product that feeds the state carries
// its inexact operands as a hi + lo pair of bf16 (x = bf16(x) + bf16(x -
// bf16(x)), 2^-16 relative): To diag(beta) and To diag(sw) in U and W, W and
// S in D = U - W S, and (fk D) in the state update, each as hi*hi + hi*lo +
// lo*hi. With decays near 1 the chunk's W S nearly cancels U, and single
// bf16 roundings there would grow the state error past 1e-3 within a few
// thousand tokens. The output-only products (Q S, P D) use single bf16.
//
// The prep writes the records with nontemporal stores: each is read once,
// by the scan, after the whole prep has run (layer prefill at config 4:
// 258 -> 242 us, most of it in the scan's reads of them).
//
// Kernel 1 (deltanet_chunk_prep_kernel): one workgroup per (chunk, value
//   head, sequence), fully parallel, three per CU (two with split inputs).
//   K and Q tiles arrive by DMA, V rows wait in registers for the A space;
//   it writes W, K^T, P, U and the row factors to the workspace, each
//   in the register order of the scan's MFMA operands (16-byte loads there).
// Kernel 2 (deltanet_chunk_scan_kernel): one 8-wave workgroup per (16-column
//   slab of dv, value head, sequence); walks the chunks in order with its
//   [dk x 16] state slab in registers (C layout of v_mfma_f32_16x16x32) of
//   four "state" waves while four "output" waves form the outputs beside
//   them; each wave prefetches its own operands of chunk c+2 into registers
//   while chunk c computes, and D and S are exchanged through LDS.
//
// Token/key "slot" order: every MFMA that contracts over an index whose
// B operand is published from C-layout registers (the state rows, the
// tokens of D) uses, within each 32-wide k-step, the order in which lane
// group g (= lane / 16) supplies k = {4g..4g+3, 16+4g..16+4g+3}. The
// workspace stores W (over k), K^T and P (over tokens) in that order.
#include "common.hpp"
#include "deltanet_generic.hpp"

#include <type_traits>

namespace aila {
namespace {

constexpr int kC = 64;          // chunk length
constexpr int kThreads = 256;
constexpr int kNumXcd = 8;      // MI355X: 8 accelerator complex dies, one L2 each

// Index held by slot e (0..7) of lane group g within a 32-wide k-step.
__device__ __forceinline__ int slot_idx(int g, int e) { return (e < 4) ? 4 * g + e : 16 + 4 * g + (e - 4); }

__device__ __forceinline__ bf16x8_t cat8x2(const u32x2& a, const u32x2& b) {
  const u32x4 r = {a[0], a[1], b[0], b[1]};
  return as_bf16x8(r);
}

// 16-byte chunk swizzles of 256-byte LDS rows (see gqa_prefill: bit 0 from
// row bit 0 suits ds_read_b128 row reads; bit 0 from row bit 3 suits the
// transposed reads).
__device__ __forceinline__ int swz_rows(int r) { return r & 15; }
__device__ __forceinline__ int swz_tr(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }

// Workspace records of one chunk. Every scan operand is stored in register
// order - [tile][k-step][lane][16 bytes] - so that one wave load is one
// contiguous KiB (a 16-row gather would cost the memory pipe 16 cache lines
// per instruction). The parts that depend on the value head (its gates)
// are kept per (sequence, value head, chunk):
//   F  fq[C], fk[C], gamma (f32)
//   W  [4 token tiles][4 k-steps][64][8 bf16]    W[16w+l%16][32ks + slots of l/16]
//   WLo  the bf16 residual W - bf16(W), laid out as W
//   P  [4 token tiles][2 k-steps][64][8 bf16]    P[16w+l%16][32s2 + slots of l/16]
//   U  [DV/16 slabs][4 token tiles][64][4 f32]   C layout of U
// and the parts that are copies of the key head's inputs once per
// (sequence, key head, chunk), written by the key head's first value head
// and read by all of them:
//   Kt [8 key tiles][2 token k-steps][64][8 bf16] K[32s2 + slots of l/16][16dt+l%16]
//   Q  [4 token tiles][4 k-steps][64][8 bf16]    Q[16w+l%16][32ks + slots of l/16]
//   KtLo (split inputs only) the bf16 residual K - bf16(K), laid out as Kt
// The key-head records follow all value-head records; the workspace sizes
// them for Hv key heads (Hk <= Hv), so its size does not depend on Hk.
template <int DK, int DV>
struct ChunkRec {
  static constexpr size_t kF = 0;
  static constexpr size_t kW = 1024;
  static constexpr size_t kWLo = kW + size_t(kC) * DK * 2;
  static constexpr size_t kP = kWLo + size_t(kC) * DK * 2;
  static constexpr size_t kU = kP + size_t(kC) * kC * 2;
  static constexpr size_t kBytes = (kU + size_t(kC) * DV * 4 + 255) / 256 * 256;
};
template <int DK, bool kLo = false>
struct KeyRec {
  static constexpr size_t kKt = 0;
  static constexpr size_t kQ = kKt + size_t(DK) * kC * 2;
  static constexpr size_t kKtLo = kQ + size_t(kC) * DK * 2;
  static constexpr size_t kBytes = (kKtLo + (kLo ? size_t(DK) * kC * 2 : 0) + 255) / 256 * 256;
};
// Key-head record (b, hk, c) of a workspace laid out for B, Hv, nch.
template <int DK, int DV, bool kLo>
__host__ __device__ __forceinline__ size_t key_rec_offset(int b, int hk, int c, int B, int Hk, int Hv, int nch) {
  return static_cast<size_t>(B) * Hv * nch * ChunkRec<DK, DV>::kBytes +
         ((static_cast<size_t>(b) * Hk + hk) * nch + c) * KeyRec<DK, kLo>::kBytes;
}

// ---------------------------------------------------------------------------
// kLo: the inputs are fp32 values carried as bf16 hi planes (q, k, v) plus
// bf16 residual tiles (q_lo, k_lo, v_lo), formed in the prep from the conv
// of the fused rows (ConvIn). The residuals enter exactly where
// the rounding of an input would reach the state beyond fp32 accuracy - the
// key norms, U (its MFMA pass and diagonal term) and the K^T operand of the
// state update (a KtLo record) - and where it would reach the outputs of
// rows whose q.k nearly cancels (the gated RMSNorm after the layer then
// magnifies an output far below sqrt(eps)): P = Q K^T takes Q_hi K_hi +
// Q_hi K_lo + Q_lo K_hi and the scan's Q S takes S as hi + lo. K K^T and W
// use the hi planes.
template <int DK, int DV, bool kLo>
__global__ __launch_bounds__(kThreads, 2) void deltanet_chunk_prep_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    ConvIn cv,
    const bf16* __restrict__ a, const bf16* __restrict__ bg, int ab_stride, const bf16* __restrict__ dt_bias,
    const float* __restrict__ A_log, unsigned char* __restrict__ ws, int T, int Hk, int Hv,
    float eps) {
  using R = ChunkRec<DK, DV>;
  using RK = KeyRec<DK, kLo>;
  static_assert(DK == 128 && DV == 128, "tiles of 64 rows x 256 bytes");
  constexpr int RB = DK * 2;       // bytes per K/Q/V row
  constexpr int NC = DK / 8;       // 16-byte chunks per row
  __shared__ __attribute__((aligned(1024))) unsigned char sK[kC * RB];    // K, swz_rows
  __shared__ __attribute__((aligned(1024))) unsigned char sQA[kC * RB];   // Q (swz_rows), then A fp32 [64][64]
  // V (swz_tr) for the split inputs; without them V waits in registers
  // until the A space frees up, which keeps the workgroup at 49.5 KiB of
  // LDS (three per CU)
  __shared__ __attribute__((aligned(1024))) unsigned char sVW[kLo ? kC * RB : 16];
  __shared__ __attribute__((aligned(16))) float sT[kC * kC];              // To, fp32 [64][64]
  __shared__ __attribute__((aligned(16))) float sG2[kC], sGn[kC], sBeta[kC], sIk[kC], sIq[kC], sSw[kC];
  float* sA = reinterpret_cast<float*>(sQA);
  unsigned char* const sV = kLo ? sVW : sQA;   // the V tile for U (transposed swizzle)
  unsigned char* sKl = reinterpret_cast<unsigned char*>(sT);   // K residual (split inputs), steps 1-3

  const int c = blockIdx.x, hv = blockIdx.y, b = blockIdx.z;
  const int nch = (T + kC - 1) / kC;
  const int hk = hv / (Hv / Hk);
  const int t0 = c * kC;
  const int n = min(kC, T - t0);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int m16 = lane & 15, g4 = lane >> 4;
  unsigned char* rec = ws + ((static_cast<size_t>(b) * Hv + hv) * nch + c) * R::kBytes;
  // the key head's first value head writes the key-head record
  const bool key_writer = hv % (Hv / Hk) == 0;
  unsigned char* krec = ws + key_rec_offset<DK, DV, kLo>(b, hk, c, static_cast<int>(gridDim.z), Hk, Hv, nch);

  // ---- 1. K, Q, V tiles (rows past T are zero) ---------------------------------
  // Split inputs (the layer): thread (cc, r0) forms 16-byte chunk cc of rows
  // r0 .. r0+3 of each tile: conv of the 7 raw rows r0-3 .. r0+3 (rows
  // before token 0 from the ring), SiLU, then bf16 hi and residual. Q, K and
  // the K residual go to their tiles now; V, its residual and a second copy
  // of the K residual wait in registers for buffers that free up later.
  const int cc1 = tid & 15, r01 = (tid >> 4) * 4;
  u32x4 vh1[4], vl1[4], kl1[4];
  auto put_rows = [&](unsigned char* tile, bool trswz, const u32x4 (&x)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = r01 + i;
      *reinterpret_cast<u32x4*>(tile + r * RB + ((cc1 ^ (trswz ? swz_tr(r) : swz_rows(r))) << 4)) = x[i];
    }
  };
  if constexpr (kLo) {
    const int head = ((cv.head % 3) + 3) % 3;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16*>(cv.qkv + static_cast<size_t>(b) * T * cv.stride), 0, T * cv.stride * 2, kBufferRsrcWord3);
    // raw rows r0-3 .. r0+3 of 8 channels from ch0 (token rows by buffer
    // load: rows past T read as zeros; rows before token 0 from the ring)
    struct Raw { u32x4 x[7]; f32x4 rg[3][2]; };
    auto load_rows = [&](int c0, Raw& o) __attribute__((always_inline)) {
      const int ch0 = c0 + cc1 * 8;
#pragma unroll
      for (int j = 0; j < 7; ++j) {
        const int t = t0 + r01 - 3 + j;
        o.x[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (t * cv.stride + ch0) * 2, 0, 0));
      }
      if (t0 + r01 < 3) {   // only the first chunk's first rows reach back before token 0
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const int t = t0 + r01 - 3 + j;
          const float* rr = cv.ring + (static_cast<size_t>(b) * 3 + (head + 3 + (t < 0 ? t : 0)) % 3) * cv.ch + ch0;
          o.rg[j][0] = *reinterpret_cast<const f32x4*>(rr);
          o.rg[j][1] = *reinterpret_cast<const f32x4*>(rr + 4);
        }
      }
    };
    // conv (4 taps) + SiLU of those rows -> bf16 hi and residual of rows r0 .. r0+3
    auto conv_tile = [&](int c0, const Raw& in, u32x4 (&hi)[4], u32x4 (&lo)[4]) __attribute__((always_inline)) {
      const int ch0 = c0 + cc1 * 8;
      float w[8][4];
#pragma unroll
      for (int v4i = 0; v4i < 4; ++v4i) {      // 16 bytes = the taps of two channels
        const u32x4 r = *reinterpret_cast<const u32x4*>(cv.w + static_cast<size_t>(ch0) * 4 + v4i * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t word = r[e >> 1];
          w[2 * v4i + (e >> 2)][e & 3] = __uint_as_float((e & 1) ? (word & 0xffff0000u) : (word << 16));
        }
      }
      float x[7][8];
#pragma unroll
      for (int j = 0; j < 7; ++j) {
        unpack8(in.x[j], x[j]);
        if (j < 3 && t0 + r01 - 3 + j < 0) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x[j][e] = in.rg[j][0][e];
            x[j][4 + e] = in.rg[j][1][e];
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float acc = x[i][e] * w[e][0];
          acc += x[i + 1][e] * w[e][1];
          acc += x[i + 2][e] * w[e][2];
          acc += x[i + 3][e] * w[e][3];
          // SiLU from the hardware exp2 and reciprocal (about 1 ulp each,
          // far below the 2^-16 the hi + lo pair carries)
          const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-acc * kLog2e));
          y[e] = (r01 + i < n) ? acc * sg : 0.f;
        }
        const u32x4 h = {pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]), pack_bf16x2(y[4], y[5]),
                         pack_bf16x2(y[6], y[7])};
        float rsd[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          rsd[e] = y[e] - __uint_as_float((e & 1) ? (h[e >> 1] & 0xffff0000u) : (h[e >> 1] << 16));
        hi[i] = h;
        lo[i] = u32x4{pack_bf16x2(rsd[0], rsd[1]), pack_bf16x2(rsd[2], rsd[3]), pack_bf16x2(rsd[4], rsd[5]),
                      pack_bf16x2(rsd[6], rsd[7])};
      }
    };
    const int qd = Hk * DK;
    // each tile's rows are in flight while the previous tile is formed
    Raw ra, rb;
    load_rows(hk * DK, ra);
    load_rows(qd + hk * DK, rb);
    u32x4 hi1[4], lo1[4];
    conv_tile(hk * DK, ra, hi1, lo1);            // Q; its residual takes the V buffer until P is formed
    put_rows(sQA, false, hi1);
    put_rows(sVW, false, lo1);
    load_rows(2 * qd + hv * DV, ra);
    conv_tile(qd + hk * DK, rb, hi1, kl1);       // K; its residual first goes to the To buffer
    put_rows(sK, false, hi1);
    put_rows(sKl, false, kl1);
    conv_tile(2 * qd + hv * DV, ra, vh1, vl1);   // V
  } else {
    const int kq_row = Hk * DK * 2, v_row = Hv * DV * 2;   // source row strides (bytes)
    const u32x4 rk = buffer_rsrc(k + (static_cast<size_t>(b) * T + t0) * Hk * DK + hk * DK, (n - 1) * kq_row + RB);
    const u32x4 rq = buffer_rsrc(q + (static_cast<size_t>(b) * T + t0) * Hk * DK + hk * DK, (n - 1) * kq_row + RB);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16*>(v + (static_cast<size_t>(b) * T + t0) * Hv * DV + hv * DV), 0, (n - 1) * v_row + RB,
        kBufferRsrcWord3);
#pragma unroll
    for (int i = 0; i < kC * NC / kThreads; ++i) {
      const int slot = i * 4 + wave;                       // wave-contiguous KiB
      const int p = slot * 64 + lane;
      const int r = p / NC, cc = p % NC;
      dma16_to_lds(rk, r * kq_row + ((cc ^ swz_rows(r)) << 4), sK + slot * 1024);
      dma16_to_lds(rq, r * kq_row + ((cc ^ swz_rows(r)) << 4), sQA + slot * 1024);
    }
    // V rows r01 .. r01+3, chunk cc1, into registers (rows past T read as zeros)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      vh1[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, (r01 + i) * v_row + cc1 * 16, 0, 0));
  }
  // gates of this chunk (wave 0, overlapping the DMA): beta, g, prefix sum G
  if (wave == 0) {
    float beta = 0.f, g = 0.f;
    if (lane < n) {
      const size_t gi = (static_cast<size_t>(b) * T + t0 + lane) * ab_stride + hv;
      beta = 1.0f / (1.0f + expf(-bf2f(bg[gi])));
      const float dtb = dt_bias ? bf2f(dt_bias[hv]) : 0.0f;
      const float negA = A_log ? -expf(A_log[hv]) : -1.0f;
      g = softplus_f(bf2f(a[gi]) + dtb) * negA;
    }
    float G = g;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(G, off);
      if (lane >= off) G += o;
    }
    sGn[lane] = G;
    sG2[lane] = G * kLog2e;
    sBeta[lane] = beta;
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm<0>());
  __syncthreads();

  auto row_chunk = [&](const unsigned char* tile, int r, int cs) __attribute__((always_inline)) {
    return *reinterpret_cast<const u32x4*>(tile + r * RB + ((cs ^ swz_rows(r)) << 4));
  };
  // ---- 2. row norms: 4 threads per row ------------------------------------------
  {
    const int r = tid >> 2, part = tid & 3;
    float sk = 0.f, sq = 0.f;
    if constexpr (kLo) {
      // |k|^2 and |q|^2 of the fp32 key and query, hi + lo
      float hi[8], lo[8];
#pragma unroll
      for (int cc = 0; cc < NC / 4; ++cc) {
        unpack8(row_chunk(sK, r, part * (NC / 4) + cc), hi);
        unpack8(row_chunk(sKl, r, part * (NC / 4) + cc), lo);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = r < n ? hi[e] + lo[e] : 0.f;
          sk = fmaf(x, x, sk);
        }
        unpack8(row_chunk(sQA, r, part * (NC / 4) + cc), hi);
        unpack8(row_chunk(sVW, r, part * (NC / 4) + cc), lo);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = hi[e] + lo[e];
          sq = fmaf(x, x, sq);
        }
      }
    }
#pragma unroll
    for (int cc = 0; cc < NC / 4; ++cc) {
      float kf[8], qf[8];
      unpack8(row_chunk(sK, r, part * (NC / 4) + cc), kf);
      unpack8(row_chunk(sQA, r, part * (NC / 4) + cc), qf);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if constexpr (!kLo) {
          sk = fmaf(kf[e], kf[e], sk);
          sq = fmaf(qf[e], qf[e], sq);
        }
      }
    }
    sk += __shfl_xor(sk, 1);
    sk += __shfl_xor(sk, 2);
    sq += __shfl_xor(sq, 1);
    sq += __shfl_xor(sq, 2);
    if (part == 0) {
      const float ik = 1.0f / sqrtf(sk + eps);
      sIk[r] = ik;
      sIq[r] = 1.0f / sqrtf(sq + eps);
      sSw[r] = sBeta[r] * expf(sGn[r]) * ik;
    }
  }
  __syncthreads();

  // ---- 2b. Q in register order for the scan (before its tile becomes A) ------
  if (key_writer) {
    u32x4* Qout = reinterpret_cast<u32x4*>(krec + RK::kQ);
#pragma unroll
    for (int i = 0; i < kC * DK * 2 / 16 / kThreads; ++i) {
      const int o = i * kThreads + tid;             // [tile][k-step][lane]
      const int l = o & 63, ks = (o >> 6) & 3, tw = o >> 8;
      const int r = tw * 16 + (l & 15), g = l >> 4;
      const int k0 = ks * 32 + 4 * g, k1 = k0 + 16;   // slots 0..3 and 4..7
      const int a0 = r * RB + (((k0 >> 3) ^ swz_rows(r)) << 4) + ((k0 & 7) << 1);
      const int a1 = r * RB + (((k1 >> 3) ^ swz_rows(r)) << 4) + ((k1 & 7) << 1);
      const u32x2 lo = *reinterpret_cast<const u32x2*>(sQA + a0);
      const u32x2 hi = *reinterpret_cast<const u32x2*>(sQA + a1);
      __builtin_nontemporal_store(u32x4{lo[0], lo[1], hi[0], hi[1]}, &Qout[o]);
    }
  }

  // ---- 3. A = masked K K^T (LDS, fp32) and P (register order, global) -------
  // Jobs 0..9: K K^T tiles (ti >= tj). Jobs 10..17: P of token tile ti over
  // s k-step s2, formed as P^T (operands swapped) for the two s tiles 2*s2,
  // 2*s2+1, so that each lane holds the 8 values of its register-order slot.
  // Wave w takes jobs w, w+4, ...; all products first (Q is read), then the
  // epilogues.
  f32x4 acc3[5][2];
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const int job = wave + 4 * i;
    acc3[i][0] = acc3[i][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (job < 10) {
      int tl = job, ti = 0;
      while (tl > ti) { tl -= ti + 1; ++ti; }
      const int tj = tl;
#pragma unroll
      for (int ks = 0; ks < DK / 32; ++ks) {
        const bf16x8_t ki = as_bf16x8(row_chunk(sK, ti * 16 + m16, ks * 4 + g4));
        const bf16x8_t kj = as_bf16x8(row_chunk(sK, tj * 16 + m16, ks * 4 + g4));
        acc3[i][0] = mfma16x16x32(ki, kj, acc3[i][0]);
        if constexpr (kLo) {
          acc3[i][0] = mfma16x16x32(ki, as_bf16x8(row_chunk(sKl, tj * 16 + m16, ks * 4 + g4)), acc3[i][0]);
          acc3[i][0] = mfma16x16x32(as_bf16x8(row_chunk(sKl, ti * 16 + m16, ks * 4 + g4)), kj, acc3[i][0]);
        }
      }
    } else if (job < 18) {
      const int ti = (job - 10) >> 1, s2 = (job - 10) & 1;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int tj = 2 * s2 + h;
        if (tj <= ti) {
#pragma unroll
          for (int ks = 0; ks < DK / 32; ++ks) {
            const bf16x8_t kb = as_bf16x8(row_chunk(sK, tj * 16 + m16, ks * 4 + g4));
            const bf16x8_t qb = as_bf16x8(row_chunk(sQA, ti * 16 + m16, ks * 4 + g4));
            acc3[i][h] = mfma16x16x32(kb, qb, acc3[i][h]);
            if constexpr (kLo) {
              // split inputs: the rounding of q and k would otherwise reach
              // the outputs of rows whose q.k nearly cancels
              acc3[i][h] = mfma16x16x32(as_bf16x8(row_chunk(sKl, tj * 16 + m16, ks * 4 + g4)), qb, acc3[i][h]);
              acc3[i][h] = mfma16x16x32(kb, as_bf16x8(row_chunk(sVW, ti * 16 + m16, ks * 4 + g4)), acc3[i][h]);
            }
          }
        }
      }
    }
  }
  __syncthreads();   // Q is no longer read: its space becomes A
  if constexpr (kLo) put_rows(sVW, true, vh1);   // the query residual is spent: V into its buffer
  auto v4 = [&](const float* arr, int i0) __attribute__((always_inline)) { return *reinterpret_cast<const f32x4*>(arr + i0); };
  u32x4* Pout = reinterpret_cast<u32x4*>(rec + R::kP);
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const int job = wave + 4 * i;
    if (job < 10) {
      int tl = job, ti = 0;
      while (tl > ti) { tl -= ti + 1; ++ti; }
      const int tj = tl;
      const int s = tj * 16 + m16, t0r = ti * 16 + g4 * 4;
      const f32x4 bt = v4(sBeta, t0r), ikt = v4(sIk, t0r), g2t = v4(sG2, t0r);
      const float iks = sIk[s], g2s = sG2[s];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = t0r + j;
        sA[t * kC + s] = (s < t) ? bt[j] * ikt[j] * iks * fast_exp2(g2t[j] - g2s) * acc3[i][0][j] : 0.f;
      }
    } else if (job < 18) {
      const int ti = (job - 10) >> 1, s2 = (job - 10) & 1;
      const int t = ti * 16 + m16;
      const float iqt = sIq[t], g2t = sG2[t];
      float pv[8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int s0 = s2 * 32 + h * 16 + 4 * g4;
        const f32x4 iks = v4(sIk, s0), g2s = v4(sG2, s0);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          pv[4 * h + j] = (s0 + j <= t) ? iqt * iks[j] * fast_exp2(g2t - g2s[j]) * acc3[i][h][j] : 0.f;
      }
      __builtin_nontemporal_store(u32x4{pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3]),
                                              pack_bf16x2(pv[4], pv[5]), pack_bf16x2(pv[6], pv[7])}, &Pout[(ti * 2 + s2) * 64 + lane]);
    }
  }
  __syncthreads();

  // ---- 4. To = (I + A)^-1 - I ---------------------------------------------------
  // 4a. diagonal block w by substitution: lane (g4, m16) owns column m16 and
  //     the partial sums over rows m = 4*g4 .. 4*g4+3 of the block.
  {
    const int base = wave * 16, j = m16;
    float xl[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) xl[kk] = (4 * g4 + kk == j) ? 1.f : 0.f;
#pragma unroll
    for (int i = 1; i < 16; ++i) {
      const f32x4 arow = *reinterpret_cast<const f32x4*>(&sA[(base + i) * kC + base + 4 * g4]);
      float part = arow[0] * xl[0];
#pragma unroll
      for (int kk = 1; kk < 4; ++kk) part = fmaf(arow[kk], xl[kk], part);   // A[i][m] = 0 for m >= i
      const float sum = xrow4_sum(part);
      const float xi = (i > j) ? -sum : ((i == j) ? 1.f : 0.f);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        if (4 * g4 + kk == i) xl[kk] = xi;
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int i = 4 * g4 + kk;
      sT[(base + i) * kC + base + j] = (i > j) ? xl[kk] : 0.f;
    }
  }
  // strictly-upper blocks of To are zero
  for (int idx = tid; idx < kC * kC; idx += kThreads) {
    const int r = idx / kC, cc = idx % kC;
    if ((cc >> 4) > (r >> 4)) sT[idx] = 0.f;
  }
  __syncthreads();
  // 4b. off-diagonal blocks by distance d on the fp32 matrix cores:
  //     T_IJ = -(I + To_II) R,  R = sum_{M=J}^{I-1} A_IM T_MJ,  T_JJ = I + To_JJ.
  // 16x16x16 products on v_mfma_f32_16x16x4f32 with the k index permuted so
  // that at step kk lane group g supplies k = 4g + kk: the A operand of the
  // four steps is one float4 of row m16, and a 16x16 block held in C layout
  // (lane (g, m16) has rows 4g..4g+3 of column m16) is directly the B
  // operand of the four steps.
  auto prod = [&](f32x4 acc, const float* X, int xr, int xc, const f32x4& yb) __attribute__((always_inline)) {
    const f32x4 xa = *reinterpret_cast<const f32x4*>(&X[(xr + m16) * kC + xc + 4 * g4]);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[kk], yb[kk], acc, 0, 0, 0);
    return acc;
  };
  auto cblock = [&](const float* Y, int yr, int yc) __attribute__((always_inline)) {   // C layout of a block
    f32x4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = Y[(yr + 4 * g4 + j) * kC + yc + m16];
    return r;
  };
  for (int d = 1; d < 4; ++d) {
    if (wave < 4 - d) {
      const int J = wave, I = J + d;
      f32x4 r = cblock(sA, I * 16, J * 16);                                 // A_IJ (identity part of T_JJ)
      r = prod(r, sA, I * 16, J * 16, cblock(sT, J * 16, J * 16));          // + A_IJ To_JJ
      for (int M = J + 1; M < I; ++M) r = prod(r, sA, I * 16, M * 16, cblock(sT, M * 16, J * 16));
      const f32x4 tr = prod(r, sT, I * 16, I * 16, r);                      // R + To_II R
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) sT[(I * 16 + 4 * g4 + jj) * kC + J * 16 + m16] = -tr[jj];
    }
    __syncthreads();
  }
  // The A space is free once To is formed: the V residual (split inputs)
  // or V itself goes there
  if constexpr (kLo) put_rows(sQA, true, vl1);
  else put_rows(sQA, true, vh1);
  __syncthreads();

  // ---- 5. U = bf16(To diag(beta)) V + diag(beta) V, then W likewise with K ----
  // wave w owns token tile w; A operands in slot order over s, B operands by
  // transposing reads of the V / K tiles in the same order.
  const int ti = wave;
  const int nks = ti / 2 + 1;                     // k-steps of 32 tokens up to the diagonal
  // (To diag(fac)) in slot order as a hi + lo pair of bf16 operands
  auto a_operand = [&](int ks, const float* fac, bf16x8_t& hi, bf16x8_t& lo) __attribute__((always_inline)) {
    const int t = ti * 16 + m16;
    float f[8], r[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int s = ks * 32 + slot_idx(g4, e);
      f[e] = sT[t * kC + s] * fac[s];
    }
    const u32x4 w = {pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7])};
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = f[e] - __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
    const u32x4 wl = {pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]), pack_bf16x2(r[4], r[5]), pack_bf16x2(r[6], r[7])};
    hi = as_bf16x8(w);
    lo = as_bf16x8(wl);
  };
  auto b_operand = [&](const unsigned char* tile, bool trswz, int ks, int dt) __attribute__((always_inline)) {
    const int d = dt * 16 + 4 * (m16 & 3);
    const int r0 = ks * 32 + 4 * g4 + (m16 >> 2), r1 = r0 + 16;
    const int z0 = trswz ? swz_tr(r0) : swz_rows(r0), z1 = trswz ? swz_tr(r1) : swz_rows(r1);
    const u32x2 lo = ds_read_tr4(tile + r0 * RB + (((d >> 3) ^ z0) << 4) + ((d & 7) << 1));
    const u32x2 hi = ds_read_tr4(tile + r1 * RB + (((d >> 3) ^ z1) << 4) + ((d & 7) << 1));
    const u32x4 w = {lo[0], lo[1], hi[0], hi[1]};
    return as_bf16x8(w);
  };
  {
    bf16x8_t au[2], aul[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      if (ks < nks) a_operand(ks, sBeta, au[ks], aul[ks]);
    float* Uout = reinterpret_cast<float*>(rec + R::kU);
#pragma unroll
    for (int dt = 0; dt < DV / 16; ++dt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        if (ks < nks) {
          const bf16x8_t vb = b_operand(sV, true, ks, dt);
          acc = mfma16x16x32(au[ks], vb, acc);
          acc = mfma16x16x32(aul[ks], vb, acc);
          if constexpr (kLo) acc = mfma16x16x32(au[ks], b_operand(sQA, true, ks, dt), acc);
        }
      // diagonal term: one transposing read gives V[ti*16 + 4*g4 + j][dt*16 + m16], j = 0..3
      const int vr = ti * 16 + 4 * g4 + (m16 >> 2), vd = dt * 16 + 4 * (m16 & 3);
      const int voff = vr * RB + (((vd >> 3) ^ swz_tr(vr)) << 4) + ((vd & 7) << 1);
      const u32x2 vv = ds_read_tr4(sV + voff);
      u32x2 vl = {0u, 0u};
      if constexpr (kLo) vl = ds_read_tr4(sQA + voff);
      const f32x4 bt = v4(sBeta, ti * 16 + g4 * 4);
      f32x4 u;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float vf = __uint_as_float((j & 1) ? (vv[j >> 1] & 0xffff0000u) : (vv[j >> 1] << 16));
        if constexpr (kLo) vf += __uint_as_float((j & 1) ? (vl[j >> 1] & 0xffff0000u) : (vl[j >> 1] << 16));
        u[j] = acc[j] + bt[j] * vf;
      }
      __builtin_nontemporal_store(u, reinterpret_cast<f32x4*>(&Uout[((dt * 4 + ti) * 64 + lane) * 4]));
    }
  }
  if constexpr (kLo) {
    __syncthreads();                        // every wave is done with V
    put_rows(sVW, false, kl1);              // K residual again (its first copy was overwritten by To)
    __syncthreads();
  }
  // W^T (operands swapped: A = K^T by transposing reads, B = (To diag(sw))^T):
  // the C layout gives lane (g4, m16) W[t = 16*tile + m16][d = 16*dt + 4*g4 + j],
  // and d tiles 2*ks, 2*ks+1 together are its register-order slot of k-step ks.
  {
    const int t = ti * 16 + m16;
    bf16x8_t bw[2], bwl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      if (ks < nks) a_operand(ks, sSw, bw[ks], bwl[ks]);
    const float swt = sSw[t];
    u32x4* Wout = reinterpret_cast<u32x4*>(rec + R::kW);
    u32x4* WLout = reinterpret_cast<u32x4*>(rec + R::kWLo);
#pragma unroll
    for (int kso = 0; kso < DK / 32; ++kso) {
      float wv[8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int dt = 2 * kso + h;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          if (ks < nks) {
            const bf16x8_t kb = b_operand(sK, false, ks, dt);
            acc = mfma16x16x32(kb, bw[ks], acc);
            acc = mfma16x16x32(kb, bwl[ks], acc);
            if constexpr (kLo) acc = mfma16x16x32(b_operand(sVW, false, ks, dt), bw[ks], acc);
          }
        const int d = dt * 16 + 4 * g4;
        const int koff = t * RB + (((d >> 3) ^ swz_rows(t)) << 4) + ((d & 7) << 1);
        const u32x2 kk = *reinterpret_cast<const u32x2*>(sK + koff);
        u32x2 kl = {0u, 0u};
        if constexpr (kLo) kl = *reinterpret_cast<const u32x2*>(sVW + koff);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float kf = __uint_as_float((j & 1) ? (kk[j >> 1] & 0xffff0000u) : (kk[j >> 1] << 16));
          if constexpr (kLo) kf += __uint_as_float((j & 1) ? (kl[j >> 1] & 0xffff0000u) : (kl[j >> 1] << 16));
          wv[4 * h + j] = acc[j] + swt * kf;
        }
      }
      const u32x4 wh = {pack_bf16x2(wv[0], wv[1]), pack_bf16x2(wv[2], wv[3]), pack_bf16x2(wv[4], wv[5]),
                        pack_bf16x2(wv[6], wv[7])};
      float wr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) wr[e] = wv[e] - __uint_as_float((e & 1) ? (wh[e >> 1] & 0xffff0000u) : (wh[e >> 1] << 16));
      __builtin_nontemporal_store(wh, &Wout[(ti * 4 + kso) * 64 + lane]);
      __builtin_nontemporal_store(u32x4{pack_bf16x2(wr[0], wr[1]), pack_bf16x2(wr[2], wr[3]),
                                                pack_bf16x2(wr[4], wr[5]), pack_bf16x2(wr[6], wr[7])}, &WLout[(ti * 4 + kso) * 64 + lane]);
    }
  }
  // ---- 6. K^T in slot order over tokens, straight from transposing reads --------
  if (key_writer) {
    bf16* Ktout = reinterpret_cast<bf16*>(krec + RK::kKt);
    // 2 token k-steps x DK/16 key tiles = 16 jobs, 4 per wave
#pragma unroll
    for (int i = 0; i < 2 * (DK / 16) / 4; ++i) {
      const int job = wave * (2 * (DK / 16) / 4) + i;
      const int ks = job & 1, dt = job >> 1;
      const bf16x8_t op = b_operand(sK, false, ks, dt);   // K[tokens in slot order][dt*16 + m16]
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, op), reinterpret_cast<u32x4*>(&Ktout[((dt * 2 + ks) * 64 + lane) * 8]));
      if constexpr (kLo) {
        const bf16x8_t ol = b_operand(sVW, false, ks, dt);
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4, ol),
                                    reinterpret_cast<u32x4*>(krec + RK::kKtLo + ((dt * 2 + ks) * 64 + lane) * 16));
      }
    }
  }
  // ---- 7. row factors --------------------------------------------------------
  float* F = reinterpret_cast<float*>(rec + R::kF);
  if (tid < kC) {
    const float Glast = sGn[n - 1];
    F[tid] = (tid < n) ? expf(sGn[tid]) * sIq[tid] : 0.f;            // fq
    F[kC + tid] = (tid < n) ? expf(Glast - sGn[tid]) * sIk[tid] : 0.f;  // fk
    if (tid == 0) F[2 * kC] = expf(Glast);                          // gamma
  }
}

// ---------------------------------------------------------------------------
// Per-chunk operands in registers (loaded two chunks ahead), by wave role.
struct StateOps {
  u32x4 w[4];        // W rows of token tile w4, k-steps 0..3 (slot order)
  u32x4 wl[4];       // residual of W
  u32x4 kt[2][2];    // K^T rows [key tile][token k-step]
  f32x4 u;           // U (C layout)
  f32x4 fk;          // fk of the 4 rows this lane holds
  float gam;
};
struct OutOps {
  u32x4 q[4];        // Q rows of token tile w4, k-steps 0..3 (slot order)
  u32x4 p[2];        // P rows, token k-steps 0..1
  f32x4 fq;
};

// One workgroup = 8 waves on one (16-column slab, value head, sequence).
// Waves 0-3 ("state" waves) carry the recurrence: each holds 32 key rows
// of the slab's state and, per chunk, computes D = U - W S for token tile
// w4, publishes D, then S = gamma S + K^T (fk D) for its key rows and
// publishes S. Waves 4-7 ("output" waves) compute O = fq (Q S) + P D for
// token tile w4 and store it. With two waves per SIMD the output path runs
// beside the state path; the chunk's two barriers order both:
//   A: state: W S, D, publish D        | output: Q S (S of this chunk)
//   B: state: K^T (fk D), publish S'   | output: + P D, store
template <int DK, int DV, bool kLo>
__global__ __launch_bounds__(2 * kThreads, 1) void deltanet_chunk_scan_kernel(
    const bf16* __restrict__ q, const unsigned char* __restrict__ ws, float* __restrict__ state,
    bf16* __restrict__ out, int T, int Hk, int Hv, float scale) {
  using R = ChunkRec<DK, DV>;
  using RK = KeyRec<DK, kLo>;
  static_assert(DK == 4 * 32, "the four state waves own 32 key rows each");
  // XCD-aware placement: workgroups are dispatched round-robin over the 8
  // XCDs, so linear id i runs on XCD i % 8. All DV/16 slabs of one head are
  // put on the same XCD, where they share the head's chunk records in L2
  // (otherwise every XCD fetches them from HBM), and each XCD takes a
  // contiguous range of heads, so that the value heads of a key head also
  // share its key-head records there.
  constexpr int kSlabs = DV / 16;
  const int nhead = static_cast<int>(gridDim.y * gridDim.z);
  const int lin = blockIdx.x + kSlabs * (blockIdx.y + static_cast<int>(gridDim.y) * blockIdx.z);
  int slab = blockIdx.x, headlin = blockIdx.y + static_cast<int>(gridDim.y) * blockIdx.z;
  if (kSlabs == kNumXcd && nhead % kNumXcd == 0) {
    const int xcd = lin % kNumXcd, i = lin / kNumXcd;
    slab = i % kSlabs;
    headlin = xcd * (nhead / kNumXcd) + i / kSlabs;
  }
  const int hv = headlin % Hv, b = headlin / Hv;
  const int nch = (T + kC - 1) / kC;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int w4 = wave & 3;
  const int m16 = lane & 15, g4 = lane >> 4;
  const int col = slab * 16 + m16;

  __shared__ u32x4 sS[4][64];            // S B-operands, one per 32-row k-step
  __shared__ u32x4 sSl[4][64];           // residual of S
  __shared__ u32x2 sD[2][2][64];         // D (bf16) B-operands: [k-step][half][lane]
  __shared__ u32x2 sDh[2][2][64];        // (fk D) hi
  __shared__ u32x2 sDl[2][2][64];        // (fk D) lo

  const unsigned char* recs = ws + (static_cast<size_t>(b) * Hv + hv) * nch * R::kBytes;
  auto rec_of = [&](int c) __attribute__((always_inline)) { return recs + static_cast<size_t>(c) * R::kBytes; };
  const unsigned char* krecs =
      ws + key_rec_offset<DK, DV, kLo>(b, hv / (Hv / Hk), 0, static_cast<int>(gridDim.z), Hk, Hv, nch);
  auto krec_of = [&](int c) __attribute__((always_inline)) { return krecs + static_cast<size_t>(c) * RK::kBytes; };

  if (wave < 4) {
    // ------------------------------------------------------------ state waves
    // Operands of a chunk in eight parts (0-3: W and W_lo of k-step p;
    // 4-5: K^T of key tile p-4; 7: U and the factors; 6 is empty - the K^T
    // residual of split inputs is loaded by its own chunk, half a chunk
    // ahead of its use, which keeps that variant within the register file).
    // The parts are issued one per MFMA group of an earlier chunk, in an
    // order that differs between slabs (below).
    auto load = [&](int c, StateOps& o, int part) __attribute__((always_inline)) {
      const unsigned char* rec = rec_of(c);
      if (part < 4) {
        o.w[part] = reinterpret_cast<const u32x4*>(rec + R::kW)[(w4 * 4 + part) * 64 + lane];
        o.wl[part] = reinterpret_cast<const u32x4*>(rec + R::kWLo)[(w4 * 4 + part) * 64 + lane];
      } else if (part < 6) {
        const int tt = part - 4;
        const u32x4* Kt = reinterpret_cast<const u32x4*>(krec_of(c) + RK::kKt) + lane;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) o.kt[tt][s2] = Kt[((w4 * 2 + tt) * 2 + s2) * 64];
      } else if (part == 6) {
        // (the K^T residual of split inputs is loaded by the chunk itself)
      } else {
        o.u = *reinterpret_cast<const f32x4*>(rec + R::kU + ((slab * 4 + w4) * 64 + lane) * 16);
        const float* F = reinterpret_cast<const float*>(rec + R::kF);
        o.fk = *reinterpret_cast<const f32x4*>(F + kC + w4 * 16 + g4 * 4);
        o.gam = F[2 * kC];
      }
    };
    // state slab in C layout: rows 32*w4 + 16*tt + 4*g4 + j, column col
    float* Sg = state + (static_cast<size_t>(b) * Hv + hv) * DK * DV;
    float s_reg[2][4];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int j = 0; j < 4; ++j) s_reg[tt][j] = Sg[static_cast<size_t>(w4 * 32 + tt * 16 + g4 * 4 + j) * DV + col];
    auto publish_state = [&]() __attribute__((always_inline)) {
      const u32x4 w = {pack_bf16x2(s_reg[0][0], s_reg[0][1]), pack_bf16x2(s_reg[0][2], s_reg[0][3]),
                       pack_bf16x2(s_reg[1][0], s_reg[1][1]), pack_bf16x2(s_reg[1][2], s_reg[1][3])};
      float r[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        r[e] = s_reg[e >> 2][e & 3] - __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
      sS[w4][lane] = w;
      sSl[w4][lane] = u32x4{pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]), pack_bf16x2(r[4], r[5]),
                            pack_bf16x2(r[6], r[7])};
    };
    // `active` is uniform; an inactive chunk (past the last one, padding the
    // three-chunk rotation) computes on repeated operands but keeps its state
    // (a select, so the chunk body stays one basic block for the schedule).
    // ROT: this slab's rotation of the load order (see the loop below).
    auto chunk = [&](bool active, const StateOps& o, int cc, int cn, StateOps& on, auto rot_c) __attribute__((always_inline)) {
      // split inputs: the K^T residual of this chunk, loaded now (half a
      // chunk ahead of its use) instead of in the rotating sets
      u32x4 ktl[2][2];
      if constexpr (kLo) {
        const u32x4* Ktl = reinterpret_cast<const u32x4*>(krec_of(min(cc, nch - 1)) + RK::kKtLo) + lane;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) ktl[tt][s2] = Ktl[((w4 * 2 + tt) * 2 + s2) * 64];
      }
      constexpr int ROT = decltype(rot_c)::value;
      // A: D = U - W S (hi*hi + hi*lo + lo*hi), published as bf16 and as
      //    hi/lo bf16 of fk D
      {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < DK / 32; ++ks) {
        const bf16x8_t sh = as_bf16x8(sS[ks][lane]);
        acc = mfma16x16x32(as_bf16x8(o.w[ks]), sh, acc);
        acc = mfma16x16x32(as_bf16x8(o.w[ks]), as_bf16x8(sSl[ks][lane]), acc);
        acc = mfma16x16x32(as_bf16x8(o.wl[ks]), sh, acc);
        load(cn, on, (ks + 2 * ROT) & 7);
        __builtin_amdgcn_sched_barrier(0);
      }
      {
        float dval[4], dsc[4], lo[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dval[j] = o.u[j] - acc[j];
          dsc[j] = o.fk[j] * dval[j];
        }
        const int s2 = w4 >> 1, half = w4 & 1;
        sD[s2][half][lane] = u32x2{pack_bf16x2(dval[0], dval[1]), pack_bf16x2(dval[2], dval[3])};
        const u32x2 hp = {pack_bf16x2(dsc[0], dsc[1]), pack_bf16x2(dsc[2], dsc[3])};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          lo[j] = dsc[j] - __uint_as_float((j & 1) ? (hp[j >> 1] & 0xffff0000u) : (hp[j >> 1] << 16));
        sDh[s2][half][lane] = hp;
        sDl[s2][half][lane] = u32x2{pack_bf16x2(lo[0], lo[1]), pack_bf16x2(lo[2], lo[3])};
      }
      }
      phase_barrier();
      // B: S = gamma S + K^T (fk D) for the key rows of this wave
      {
      bf16x8_t dh[2], dl[2];
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        dh[s2] = cat8x2(sDh[s2][0][lane], sDh[s2][1][lane]);
        dl[s2] = cat8x2(sDl[s2][0][lane], sDl[s2][1][lane]);
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        f32x4 a2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const bf16x8_t aK = as_bf16x8(o.kt[tt][s2]);
          a2 = mfma16x16x32(aK, dh[s2], a2);
          a2 = mfma16x16x32(aK, dl[s2], a2);
          if constexpr (kLo) a2 = mfma16x16x32(as_bf16x8(ktl[tt][s2]), dh[s2], a2);
          load(cn, on, (4 + 2 * tt + s2 + 2 * ROT) & 7);
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) s_reg[tt][j] = active ? o.gam * s_reg[tt][j] + a2[j] : s_reg[tt][j];
      }
      publish_state();
      }
      phase_barrier();
    };
    publish_state();
    // Three operand sets rotate; loads are unconditional (clamped to the
    // last chunk) so that the compiler's wait counts stay exact.
    // The slabs of a head read the same chunk records at about the same
    // time; each group of slabs issues the parts in a different order, so
    // that their requests meet fewer times on one L2 channel (config 4:
    // 171 -> 160 us; layer prefill 271 -> 258 us).
    auto run = [&](auto rot_c) __attribute__((always_inline)) {
      StateOps o0, o1, o2;
#pragma unroll
      for (int part = 0; part < 8; ++part) load(0, o0, part);
#pragma unroll
      for (int part = 0; part < 8; ++part) load(min(1, nch - 1), o1, part);
      __syncthreads();
      for (int c = 0; c < nch; c += 3) {
        chunk(true, o0, c, min(c + 2, nch - 1), o2, rot_c);
        chunk(c + 1 < nch, o1, c + 1, min(c + 3, nch - 1), o0, rot_c);
        chunk(c + 2 < nch, o2, c + 2, min(c + 4, nch - 1), o1, rot_c);
      }
    };
    switch (slab & 3) {
      case 0: run(std::integral_constant<int, 0>{}); break;
      case 1: run(std::integral_constant<int, 1>{}); break;
      case 2: run(std::integral_constant<int, 2>{}); break;
      default: run(std::integral_constant<int, 3>{}); break;
    }
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int j = 0; j < 4; ++j) Sg[static_cast<size_t>(w4 * 32 + tt * 16 + g4 * 4 + j) * DV + col] = s_reg[tt][j];
  } else {
    // ----------------------------------------------------------- output waves
    // parts 0-3: Q of k-step p; 4: P and fq (interleaved as in the state waves)
    auto load = [&](int c, OutOps& o, int part) __attribute__((always_inline)) {
      const unsigned char* rec = rec_of(c);
      if (part < 4) {
        o.q[part] = reinterpret_cast<const u32x4*>(krec_of(c) + RK::kQ)[(w4 * 4 + part) * 64 + lane];
      } else {
        const u32x4* P = reinterpret_cast<const u32x4*>(rec + R::kP) + w4 * 2 * 64 + lane;
        o.p[0] = P[0];
        o.p[1] = P[64];
        o.fq = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(rec + R::kF) + w4 * 16 + g4 * 4);
      }
    };
    // Output rows go out through a buffer resource bounded at the chunk's
    // last token, so the stores need no per-row branch (rows past T drop).
    const int rs2 = Hv * DV * 2;   // bytes per token row
    const int lane_off = ((w4 * 16 + g4 * 4) * Hv + hv) * DV * 2 + col * 2;
    auto chunk = [&](bool active, int c, const OutOps& o, int cn, OutOps& on, auto rot_c) __attribute__((always_inline)) {
      constexpr int ROT = decltype(rot_c)::value;
      // A: Q S with the state of this chunk
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < DK / 32; ++ks) {
        const bf16x8_t sh = as_bf16x8(sS[ks][lane]);
        acc = mfma16x16x32(as_bf16x8(o.q[ks]), sh, acc);
        // split inputs: S as hi + lo (the residual of Q adds ~15% to the
        // scan's operand bytes for no measurable gain: P carries it)
        if constexpr (kLo) acc = mfma16x16x32(as_bf16x8(o.q[ks]), as_bf16x8(sSl[ks][lane]), acc);
        load(cn, on, (ks + ROT) % 5);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] *= o.fq[j];
      phase_barrier();
      // B: + P D, store (an inactive chunk's resource holds no bytes)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
        if (s2 <= (w4 >> 1)) acc = mfma16x16x32(as_bf16x8(o.p[s2]), cat8x2(sD[s2][0][lane], sD[s2][1][lane]), acc);
      load(cn, on, (4 + ROT) % 5);
      const int t0 = min(c, nch - 1) * kC;
      const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(
          out + (static_cast<size_t>(b) * T + t0) * Hv * DV, 0, active ? min(kC, T - t0) * rs2 : 0, kBufferRsrcWord3);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        __builtin_amdgcn_raw_buffer_store_b16(f2bf(scale * acc[j]), orsrc, lane_off + j * rs2, 0, 0);
      phase_barrier();
    };
    auto run = [&](auto rot_c) __attribute__((always_inline)) {   // load orders as in the state waves
      OutOps o0, o1, o2;
#pragma unroll
      for (int part = 0; part < 5; ++part) load(0, o0, part);
#pragma unroll
      for (int part = 0; part < 5; ++part) load(min(1, nch - 1), o1, part);
      __syncthreads();
      for (int c = 0; c < nch; c += 3) {
        chunk(true, c, o0, min(c + 2, nch - 1), o2, rot_c);
        chunk(c + 1 < nch, c + 1, o1, min(c + 3, nch - 1), o0, rot_c);
        chunk(c + 2 < nch, c + 2, o2, min(c + 4, nch - 1), o1, rot_c);
      }
    };
    switch (slab & 3) {
      case 0: run(std::integral_constant<int, 0>{}); break;
      case 1: run(std::integral_constant<int, 1>{}); break;
      case 2: run(std::integral_constant<int, 2>{}); break;
      default: run(std::integral_constant<int, 3>{}); break;
    }
  }
}

}  // namespace
}  // namespace aila

namespace aila {
// Chunk records + launches of the two kernels; shared by the recurrence
// entry point (bf16 inputs) and the full layer (split fp32 inputs).
size_t deltanet_chunk_records_bytes(int B, int T, int Hv, bool split) {
  const size_t nch = (static_cast<size_t>(T) + kC - 1) / kC;
  return static_cast<size_t>(B) * Hv * nch *
         (ChunkRec<128, 128>::kBytes + (split ? KeyRec<128, true>::kBytes : KeyRec<128, false>::kBytes));
}

// conv == nullptr: q, k, v planes (bf16 inputs). Otherwise the layer: q, k,
// v are formed from conv->qkv by the prep (q, k, v unused).
void launch_deltanet_chunked(const bf16* q, const bf16* k, const bf16* v, const ConvIn* conv, const bf16* a,
                             const bf16* b, int ab_stride, const bf16* dt_bias, const float* A_log, float* state,
                             bf16* out, unsigned char* records, int B, int T, int Hk, int Hv, float eps, float scale,
                             hipStream_t st) {
  const int nch = (T + kC - 1) / kC;
  if (conv) {
    hipLaunchKernelGGL((deltanet_chunk_prep_kernel<128, 128, true>), dim3(nch, Hv, B), dim3(kThreads), 0, st, q, k,
                       v, *conv, a, b, ab_stride, dt_bias, A_log, records, T, Hk, Hv, eps);
    hipLaunchKernelGGL((deltanet_chunk_scan_kernel<128, 128, true>), dim3(128 / 16, Hv, B), dim3(2 * kThreads), 0,
                       st, q, records, state, out, T, Hk, Hv, scale);
  } else {
    hipLaunchKernelGGL((deltanet_chunk_prep_kernel<128, 128, false>), dim3(nch, Hv, B), dim3(kThreads), 0, st, q, k,
                       v, ConvIn{}, a, b, ab_stride, dt_bias, A_log, records, T, Hk, Hv, eps);
    hipLaunchKernelGGL((deltanet_chunk_scan_kernel<128, 128, false>), dim3(128 / 16, Hv, B), dim3(2 * kThreads), 0,
                       st, q, records, state, out, T, Hk, Hv, scale);
  }
}
}  // namespace aila

extern "C" size_t aila_hip_deltanet_prefill_workspace_size(int B, int T, int Hv, int dk, int dv) {
  // 0 also for the shapes that run the sequential general-shape kernel
  if (B <= 0 || T <= 0 || Hv <= 0 || dk != 128 || dv != 128) return 0;
  return aila::deltanet_chunk_records_bytes(B, T, Hv, false);
}

extern "C" int aila_hip_deltanet_prefill(const void* q, const void* k, const void* v, const void* a,
                                         const void* b, const void* dt_bias, const float* A_log,
                                         float* state, void* out, void* workspace,
                                         size_t workspace_bytes, int B, int T, int Hk, int Hv,
                                         int dk, int dv, float eps, float scale, void* stream) {
  using namespace aila;
  AILA_REQUIRE(q && k && v && a && b && state && out, "deltanet_prefill: null pointer");
  AILA_REQUIRE(B > 0 && B <= 65535 && T > 0 && Hk > 0 && Hv > 0 && Hv <= 65535,
               "deltanet_prefill: bad shape (B=%d T=%d Hk=%d Hv=%d)", B, T, Hk, Hv);
  if (dk != 128 || dv != 128 || Hv % Hk != 0) {
    // general shapes: the token-sequential kernel (no workspace)
    GenericDeltaNet g{};
    g.q = static_cast<const bf16*>(q);
    g.k = static_cast<const bf16*>(k);
    g.v = static_cast<const bf16*>(v);
    g.a = static_cast<const bf16*>(a);
    g.b = static_cast<const bf16*>(b);
    g.ab_stride = Hv;
    g.dt_bias = static_cast<const bf16*>(dt_bias);
    g.A_log = A_log;
    g.state = state;
    g.out = static_cast<bf16*>(out);
    g.B = B, g.T = T, g.Hk = Hk, g.Hv = Hv, g.dk = dk, g.dv = dv, g.K = 1;
    g.eps = eps, g.scale = scale;
    return deltanet_generic_launch(g, static_cast<hipStream_t>(stream), "deltanet_prefill");
  }
  const size_t need = aila_hip_deltanet_prefill_workspace_size(B, T, Hv, dk, dv);
  if (!workspace || workspace_bytes < need)
    return set_error(AILA_HIP_EWORKSPACE, "deltanet_prefill: workspace %zu < %zu bytes", workspace_bytes, need);
  launch_deltanet_chunked(static_cast<const bf16*>(q), static_cast<const bf16*>(k), static_cast<const bf16*>(v),
                          nullptr, static_cast<const bf16*>(a), static_cast<const bf16*>(b), Hv,
                          static_cast<const bf16*>(dt_bias), A_log, state, static_cast<bf16*>(out),
                          static_cast<unsigned char*>(workspace), B, T, Hk, Hv, eps, scale,
                          static_cast<hipStream_t>(stream));
  return check_launch("deltanet_prefill");
}

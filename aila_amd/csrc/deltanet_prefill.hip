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
// so they stay in [0, 1]. The diagonal of T is applied in fp32, and the
// state update K^T (fk D) uses a hi/lo bf16 split of (fk D); every other
// MFMA operand is either an exact bf16 input or a single bf16 rounding.
//
// Kernel 1 (deltanet_chunk_prep_kernel): one workgroup per (chunk, value
//   head, sequence), fully parallel. Writes W, U, P, K^T and the row
//   factors to the workspace.
// Kernel 2 (deltanet_chunk_scan_kernel): one workgroup per (16-column slab
//   of dv, value head, sequence); walks the chunks in order with its
//   [dk x 16] state slab in registers (C layout of v_mfma_f32_16x16x32),
//   exchanging MFMA operands between its 4 waves through LDS.
#include "common.hpp"

namespace aila {
namespace {

constexpr int kC = 64;          // chunk length
constexpr int kThreads = 256;

__device__ __forceinline__ float softplus_f(float x) {
  if (x > 20.0f) return x;
  if (x < -20.0f) return expf(x);
  return log1pf(expf(x));
}

// Workspace record of one (sequence, value head, chunk).
template <int DK, int DV>
struct ChunkRec {
  static constexpr size_t kW = 0;                                   // bf16 [C][DK]
  static constexpr size_t kU = kW + size_t(kC) * DK * 2;            // f32  [C][DV]
  static constexpr size_t kP = kU + size_t(kC) * DV * 4;            // bf16 [C][C]
  static constexpr size_t kKt = kP + size_t(kC) * kC * 2;           // bf16 [DK][C]
  static constexpr size_t kF = kKt + size_t(DK) * kC * 2;           // f32 fq[C], fk[C], gam
  static constexpr size_t kBytes = ((kF + (2 * kC + 16) * 4) + 255) / 256 * 256;
};

__device__ __forceinline__ u32x2 ld8(const void* p) { return *reinterpret_cast<const u32x2*>(p); }

__device__ __forceinline__ bf16x8_t cat8(const u32x2& a, const u32x2& b) {
  u32x4 r = {a[0], a[1], b[0], b[1]};
  return as_bf16x8(r);
}

// ---------------------------------------------------------------------------
template <int DK, int DV>
__global__ __launch_bounds__(kThreads) void deltanet_chunk_prep_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const bf16* __restrict__ a, const bf16* __restrict__ bg, const bf16* __restrict__ dt_bias,
    const float* __restrict__ A_log, unsigned char* __restrict__ ws, int T, int Hk, int Hv,
    float eps) {
  using R = ChunkRec<DK, DV>;
  constexpr int KP = DK + 8;       // row pitch of K/Q tiles (bf16)
  constexpr int TP = kC + 8;       // row pitch of transposed tiles (bf16)
  constexpr int AP = kC + 1;       // fp32 pitch of A / To
  __shared__ __attribute__((aligned(16))) bf16 sK[kC * KP];
  __shared__ __attribute__((aligned(16))) bf16 sQ[kC * KP];
  __shared__ __attribute__((aligned(16))) bf16 sKt[DK * TP];
  __shared__ __attribute__((aligned(16))) bf16 sVt[DV * TP];
  __shared__ float sA[kC * AP];
  __shared__ float sT[kC * AP];
  __shared__ float sR[3 * 256];
  __shared__ float sG[kC], sBeta[kC], sIk[kC], sIq[kC], sSw[kC];

  const int c = blockIdx.x, hv = blockIdx.y, b = blockIdx.z;
  const int nch = (T + kC - 1) / kC;
  const int hk = hv / (Hv / Hk);
  const int t0 = c * kC;
  const int n = min(kC, T - t0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m16 = lane & 15, g4 = lane >> 4;
  unsigned char* rec = ws + ((static_cast<size_t>(b) * Hv + hv) * nch + c) * R::kBytes;

  // ---- 1. stage K, Q (row-major), K^T, V^T ---------------------------------
  for (int idx = tid; idx < kC * (DK / 8); idx += kThreads) {
    const int r = idx / (DK / 8), c8 = idx % (DK / 8);
    u32x4 kv = {0u, 0u, 0u, 0u}, qv = {0u, 0u, 0u, 0u};
    if (r < n) {
      const size_t row = (static_cast<size_t>(b) * T + t0 + r) * Hk + hk;
      kv = ld16(k + row * DK + c8 * 8);
      qv = ld16(q + row * DK + c8 * 8);
    }
    *reinterpret_cast<u32x4*>(&sK[r * KP + c8 * 8]) = kv;
    *reinterpret_cast<u32x4*>(&sQ[r * KP + c8 * 8]) = qv;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      sKt[(c8 * 8 + e) * TP + r] = static_cast<bf16>((e & 1) ? (kv[e >> 1] >> 16) : (kv[e >> 1] & 0xffffu));
  }
  for (int idx = tid; idx < kC * (DV / 8); idx += kThreads) {
    const int r = idx / (DV / 8), c8 = idx % (DV / 8);
    u32x4 vv = {0u, 0u, 0u, 0u};
    if (r < n) vv = ld16(v + ((static_cast<size_t>(b) * T + t0 + r) * Hv + hv) * DV + c8 * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      sVt[(c8 * 8 + e) * TP + r] = static_cast<bf16>((e & 1) ? (vv[e >> 1] >> 16) : (vv[e >> 1] & 0xffffu));
  }
  // gates of this chunk (wave 0): beta, g, inclusive prefix sum G
  if (wave == 0) {
    float beta = 0.f, g = 0.f;
    if (lane < n) {
      const size_t gi = (static_cast<size_t>(b) * T + t0 + lane) * Hv + hv;
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
    sG[lane] = G;
    sBeta[lane] = beta;
  }
  __syncthreads();
  // row norms: 4 threads per row, for K and Q
  {
    const int r = tid >> 2, part = tid & 3;
    float sk = 0.f, sq = 0.f;
    for (int d = part * (DK / 4); d < (part + 1) * (DK / 4); ++d) {
      const float kf = bf2f(sK[r * KP + d]), qf = bf2f(sQ[r * KP + d]);
      sk += kf * kf;
      sq += qf * qf;
    }
    sk += __shfl_xor(sk, 1);
    sk += __shfl_xor(sk, 2);
    sq += __shfl_xor(sq, 1);
    sq += __shfl_xor(sq, 2);
    if (part == 0) {
      const float ik = 1.0f / sqrtf(sk + eps);
      sIk[r] = ik;
      sIq[r] = 1.0f / sqrtf(sq + eps);
      sSw[r] = sBeta[r] * expf(sG[r]) * ik;
    }
  }
  __syncthreads();

  // ---- 2. K K^T and Q K^T (lower tiles) on MFMA -------------------------------
  // tile list: (ti, tj) with tj <= ti: 10 tiles per product, 20 in total.
  bf16* Pout = reinterpret_cast<bf16*>(rec + R::kP);
  for (int job = wave; job < 20; job += 4) {
    const bool isq = job >= 10;
    int tl = isq ? job - 10 : job;
    int ti = 0;
    while (tl > ti) { tl -= ti + 1; ++ti; }
    const int tj = tl;
    const bf16* X = isq ? sQ : sK;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < DK / 32; ++ks) {
      const bf16x8_t av = as_bf16x8(*reinterpret_cast<const u32x4*>(&X[(ti * 16 + m16) * KP + ks * 32 + g4 * 8]));
      const bf16x8_t bv = as_bf16x8(*reinterpret_cast<const u32x4*>(&sK[(tj * 16 + m16) * KP + ks * 32 + g4 * 8]));
      acc = mfma16x16x32(av, bv, acc);
    }
    const int s = tj * 16 + m16;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = ti * 16 + g4 * 4 + j;
      if (!isq) {
        const float val = (s < t) ? sBeta[t] * expf(sG[t] - sG[s]) * sIk[t] * sIk[s] * acc[j] : 0.f;
        sA[t * AP + s] = val;
        if (ti != tj) sA[s * AP + t] = 0.f;     // upper triangle
      } else {
        const float val = (s <= t) ? expf(sG[t] - sG[s]) * sIq[t] * sIk[s] * acc[j] : 0.f;
        Pout[t * kC + s] = f2bf(val);
        if (ti != tj) Pout[s * kC + t] = 0;
      }
    }
  }
  __syncthreads();

  // ---- 3. To = (I + A)^-1 - I, blocked by 16 ----------------------------------
  // 3a. diagonal blocks: wave w, lane j < 16 owns column j of block w.
  if (m16 == lane) {   // lanes 0..15 of each wave
    const int base = wave * 16;
    const int j = lane;
    float tc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) tc[i] = 0.f;
#pragma unroll
    for (int i = 1; i < 16; ++i) {
      if (j < i) {
        float acc = sA[(base + i) * AP + base + j];
#pragma unroll
        for (int m = 1; m < 16; ++m)
          if (m > j && m < i) acc += sA[(base + i) * AP + base + m] * tc[m];
        tc[i] = -acc;
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sT[(base + i) * AP + base + j] = tc[i];
  }
  // clear the strictly-upper blocks of sT
  for (int idx = tid; idx < kC * kC; idx += kThreads) {
    const int r = idx / kC, cc = idx % kC;
    if ((cc >> 4) > (r >> 4)) sT[r * AP + cc] = 0.f;
  }
  __syncthreads();
  // 3b. off-diagonal blocks by distance d: T_IJ = -(I + To_II) R,
  //     R = sum_{M=J}^{I-1} A_IM T_MJ with T_JJ = I + To_JJ.
  for (int d = 1; d < 4; ++d) {
    const int nblk = 4 - d;
    for (int e = tid; e < nblk * 256; e += kThreads) {
      const int J = e >> 8, I = J + d;
      const int i = (e >> 4) & 15, j = e & 15;
      const int row = I * 16 + i, col = J * 16 + j;
      float acc = sA[row * AP + col];           // M = J, identity part of T_JJ
      for (int m = J * 16; m < I * 16; ++m) acc += sA[row * AP + m] * sT[m * AP + col];
      sR[e] = acc;
    }
    __syncthreads();
    for (int e = tid; e < nblk * 256; e += kThreads) {
      const int J = e >> 8, I = J + d;
      const int i = (e >> 4) & 15, j = e & 15;
      float acc = sR[e];
      for (int m = 0; m < i; ++m) acc += sT[(I * 16 + i) * AP + I * 16 + m] * sR[(J << 8) + (m << 4) + j];
      sT[(I * 16 + i) * AP + J * 16 + j] = -acc;
    }
    __syncthreads();
  }

  // ---- 4. W and U: wave w owns token tile w ---------------------------------
  {
    const int ti = wave;
    const int nks = ti / 2 + 1;     // k-steps of 32 tokens below the diagonal
    bf16x8_t aw[2], au[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if (ks < nks) {
        const int t = ti * 16 + m16;
        float wv[8], uv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int s = ks * 32 + g4 * 8 + e;
          const float tv = sT[t * AP + s];
          wv[e] = tv * sSw[s];
          uv[e] = tv * sBeta[s];
        }
        u32x4 pw = {pack_bf16x2(wv[0], wv[1]), pack_bf16x2(wv[2], wv[3]), pack_bf16x2(wv[4], wv[5]), pack_bf16x2(wv[6], wv[7])};
        u32x4 pu = {pack_bf16x2(uv[0], uv[1]), pack_bf16x2(uv[2], uv[3]), pack_bf16x2(uv[4], uv[5]), pack_bf16x2(uv[6], uv[7])};
        aw[ks] = as_bf16x8(pw);
        au[ks] = as_bf16x8(pu);
      }
    }
    bf16* Wout = reinterpret_cast<bf16*>(rec + R::kW);
    float* Uout = reinterpret_cast<float*>(rec + R::kU);
#pragma unroll
    for (int dt = 0; dt < DK / 16; ++dt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (ks < nks) {
          const bf16x8_t bv = as_bf16x8(*reinterpret_cast<const u32x4*>(&sKt[(dt * 16 + m16) * TP + ks * 32 + g4 * 8]));
          acc = mfma16x16x32(aw[ks], bv, acc);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = ti * 16 + g4 * 4 + j, dd = dt * 16 + m16;
        const float w = acc[j] + sSw[t] * bf2f(sK[t * KP + dd]);
        Wout[t * DK + dd] = f2bf(w);
      }
    }
#pragma unroll
    for (int dt = 0; dt < DV / 16; ++dt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (ks < nks) {
          const bf16x8_t bv = as_bf16x8(*reinterpret_cast<const u32x4*>(&sVt[(dt * 16 + m16) * TP + ks * 32 + g4 * 8]));
          acc = mfma16x16x32(au[ks], bv, acc);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = ti * 16 + g4 * 4 + j, dd = dt * 16 + m16;
        Uout[t * DV + dd] = acc[j] + sBeta[t] * bf2f(sVt[dd * TP + t]);
      }
    }
  }
  // ---- 5. K^T and the row factors ---------------------------------------------
  bf16* Ktout = reinterpret_cast<bf16*>(rec + R::kKt);
  for (int idx = tid; idx < DK * (kC / 8); idx += kThreads) {
    const int r = idx / (kC / 8), c8 = idx % (kC / 8);
    *reinterpret_cast<u32x4*>(&Ktout[r * kC + c8 * 8]) = *reinterpret_cast<const u32x4*>(&sKt[r * TP + c8 * 8]);
  }
  float* F = reinterpret_cast<float*>(rec + R::kF);
  if (tid < kC) {
    const float Glast = sG[n - 1];
    F[tid] = (tid < n) ? expf(sG[tid]) * sIq[tid] : 0.f;            // fq
    F[kC + tid] = (tid < n) ? expf(Glast - sG[tid]) * sIk[tid] : 0.f;  // fk
    if (tid == 0) F[2 * kC] = expf(Glast);                          // gamma
  }
}

// ---------------------------------------------------------------------------
template <int DK, int DV>
__global__ __launch_bounds__(kThreads) void deltanet_chunk_scan_kernel(
    const bf16* __restrict__ q, const unsigned char* __restrict__ ws, float* __restrict__ state,
    bf16* __restrict__ out, int T, int Hk, int Hv, float scale) {
  using R = ChunkRec<DK, DV>;
  static_assert(DK == 4 * 32, "the four waves own 32 key rows each");
  const int slab = blockIdx.x, hv = blockIdx.y, b = blockIdx.z;
  const int nch = (T + kC - 1) / kC;
  const int hk = hv / (Hv / Hk);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m16 = lane & 15, g4 = lane >> 4;
  const int col = slab * 16 + m16;

  __shared__ u32x4 sS[4][64];            // S B-operands, one per 32-row k-step
  __shared__ u32x2 sD[2][2][64];         // D (bf16) B-operands: [k-step][half][lane]
  __shared__ u32x2 sDh[2][2][64];        // (fk D) hi
  __shared__ u32x2 sDl[2][2][64];        // (fk D) lo

  // state slab in C layout: rows 32*wave + 16*tt + 4*g4 + j, column col
  float* Sg = state + (static_cast<size_t>(b) * Hv + hv) * DK * DV;
  float s_reg[2][4];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int j = 0; j < 4; ++j) s_reg[tt][j] = Sg[static_cast<size_t>(wave * 32 + tt * 16 + g4 * 4 + j) * DV + col];

  auto publish_state = [&]() {
    u32x4 w = {pack_bf16x2(s_reg[0][0], s_reg[0][1]), pack_bf16x2(s_reg[0][2], s_reg[0][3]),
               pack_bf16x2(s_reg[1][0], s_reg[1][1]), pack_bf16x2(s_reg[1][2], s_reg[1][3])};
    sS[wave][lane] = w;
  };
  publish_state();
  __syncthreads();

  for (int c = 0; c < nch; ++c) {
    const int t0 = c * kC;
    const int n = min(kC, T - t0);
    const unsigned char* rec = ws + ((static_cast<size_t>(b) * Hv + hv) * nch + c) * R::kBytes;
    const bf16* W = reinterpret_cast<const bf16*>(rec + R::kW);
    const float* U = reinterpret_cast<const float*>(rec + R::kU);
    const bf16* P = reinterpret_cast<const bf16*>(rec + R::kP);
    const bf16* Kt = reinterpret_cast<const bf16*>(rec + R::kKt);
    const float* F = reinterpret_cast<const float*>(rec + R::kF);

    // ---- D = U - W S and Q S for token tile `wave` ----------------------------
    const int trow = wave * 16 + m16;                 // A-operand row (token)
    const int tq = min(t0 + trow, T - 1);
    const bf16* qrow = q + ((static_cast<size_t>(b) * T + tq) * Hk + hk) * DK;
    f32x4 ws_acc = {0.f, 0.f, 0.f, 0.f}, qs_acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < DK / 32; ++ks) {
      const int k0 = ks * 32 + g4 * 4;
      const bf16x8_t aW = cat8(ld8(W + trow * DK + k0), ld8(W + trow * DK + k0 + 16));
      const bf16x8_t aQ = cat8(ld8(qrow + k0), ld8(qrow + k0 + 16));
      const bf16x8_t bS = as_bf16x8(sS[ks][lane]);
      ws_acc = mfma16x16x32(aW, bS, ws_acc);
      qs_acc = mfma16x16x32(aQ, bS, qs_acc);
    }
    float dval[4], dsc[4];
    f32x4 o_acc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = wave * 16 + g4 * 4 + j;
      dval[j] = U[t * DV + col] - ws_acc[j];
      dsc[j] = F[kC + t] * dval[j];
      o_acc[j] = F[t] * qs_acc[j];
    }
    // publish D (bf16) and fk*D (hi/lo) as B operands of the 32-token k-steps
    {
      const int s2 = wave >> 1, half = wave & 1;
      sD[s2][half][lane] = u32x2{pack_bf16x2(dval[0], dval[1]), pack_bf16x2(dval[2], dval[3])};
      float hi[4], lo[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hi[j] = bf2f(f2bf(dsc[j]));
        lo[j] = dsc[j] - hi[j];
      }
      sDh[s2][half][lane] = u32x2{pack_bf16x2(hi[0], hi[1]), pack_bf16x2(hi[2], hi[3])};
      sDl[s2][half][lane] = u32x2{pack_bf16x2(lo[0], lo[1]), pack_bf16x2(lo[2], lo[3])};
    }
    __syncthreads();

    // ---- O += P D ; store ---------------------------------------------------------
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      if (s2 <= (wave >> 1)) {
        const int k0 = s2 * 32 + g4 * 4;
        const bf16x8_t aP = cat8(ld8(P + trow * kC + k0), ld8(P + trow * kC + k0 + 16));
        const u32x2 lo2 = sD[s2][0][lane], hi2 = sD[s2][1][lane];
        o_acc = mfma16x16x32(aP, cat8(lo2, hi2), o_acc);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = wave * 16 + g4 * 4 + j;
      if (t < n) out[((static_cast<size_t>(b) * T + t0 + t) * Hv + hv) * DV + col] = f2bf(scale * o_acc[j]);
    }

    // ---- S = gamma S + K^T (fk D) for key rows of this wave ------------------------
    const float gam = F[2 * kC];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int krow = wave * 32 + tt * 16 + m16;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const int k0 = s2 * 32 + g4 * 4;
        const bf16x8_t aK = cat8(ld8(Kt + krow * kC + k0), ld8(Kt + krow * kC + k0 + 16));
        acc = mfma16x16x32(aK, cat8(sDh[s2][0][lane], sDh[s2][1][lane]), acc);
        acc = mfma16x16x32(aK, cat8(sDl[s2][0][lane], sDl[s2][1][lane]), acc);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) s_reg[tt][j] = gam * s_reg[tt][j] + acc[j];
    }
    publish_state();
    __syncthreads();
  }
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int j = 0; j < 4; ++j) Sg[static_cast<size_t>(wave * 32 + tt * 16 + g4 * 4 + j) * DV + col] = s_reg[tt][j];
}

}  // namespace
}  // namespace aila

extern "C" size_t aila_hip_deltanet_prefill_workspace_size(int B, int T, int Hv, int dk, int dv) {
  if (B <= 0 || T <= 0 || Hv <= 0 || dk != 128 || dv != 128) return 0;
  const size_t nch = (static_cast<size_t>(T) + aila::kC - 1) / aila::kC;
  return static_cast<size_t>(B) * Hv * nch * aila::ChunkRec<128, 128>::kBytes;
}

extern "C" int aila_hip_deltanet_prefill(const void* q, const void* k, const void* v, const void* a,
                                         const void* b, const void* dt_bias, const float* A_log,
                                         float* state, void* out, void* workspace,
                                         size_t workspace_bytes, int B, int T, int Hk, int Hv,
                                         int dk, int dv, float eps, float scale, void* stream) {
  using namespace aila;
  AILA_REQUIRE(q && k && v && a && b && state && out, "deltanet_prefill: null pointer");
  AILA_REQUIRE(B > 0 && B <= 65535 && T > 0 && Hk > 0 && Hv > 0 && Hv % Hk == 0 && Hv <= 65535,
               "deltanet_prefill: bad shape (B=%d T=%d Hk=%d Hv=%d)", B, T, Hk, Hv);
  if (dk != 128 || dv != 128)
    return set_error(AILA_HIP_EUNSUPPORTED, "deltanet_prefill: dk=%d dv=%d (only 128/128)", dk, dv);
  const size_t need = aila_hip_deltanet_prefill_workspace_size(B, T, Hv, dk, dv);
  if (!workspace || workspace_bytes < need)
    return set_error(AILA_HIP_EWORKSPACE, "deltanet_prefill: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nch = (T + kC - 1) / kC;
  hipLaunchKernelGGL((deltanet_chunk_prep_kernel<128, 128>), dim3(nch, Hv, B), dim3(kThreads), 0, st,
                     static_cast<const bf16*>(q), static_cast<const bf16*>(k), static_cast<const bf16*>(v),
                     static_cast<const bf16*>(a), static_cast<const bf16*>(b),
                     static_cast<const bf16*>(dt_bias), A_log, static_cast<unsigned char*>(workspace), T,
                     Hk, Hv, eps);
  hipLaunchKernelGGL((deltanet_chunk_scan_kernel<128, 128>), dim3(dv / 16, Hv, B), dim3(kThreads), 0, st,
                     static_cast<const bf16*>(q), static_cast<const unsigned char*>(workspace), state,
                     static_cast<bf16*>(out), T, Hk, Hv, scale);
  return check_launch("deltanet_prefill");
}

// Causal GQA prefill on bf16 MFMA (gfx950), flash-attention style.
//
// Reference: ops::attention_prefill (src/ops/AttentionOps.cpp:649-842),
// ops::attention_prefill_cached (:2308-2507) and ops::copy_to_cache
// (:2513-2532). The reference materialises an [H, S, S] fp32 score matrix
// (naive branch) or walks one query row per workgroup (D=256 branch); here a
// workgroup owns BM query rows of one head and streams K/V tiles through LDS
// with an online softmax in registers, so K/V are reused across BM rows.
//
// Orientation (the key choice for CDNA MFMA layouts):
//   S^T = K Q^T     A = K tile (LDS, key rows), B = Q^T (registers)
//                   -> lane l holds query row l%16, keys 4*(l/16)+j
//   O^T += V^T P^T  A = V^T tile (LDS, stored transposed), B = P^T straight
//                   from the S^T registers (no data movement)
// so the softmax row statistics of a query row live in the four lanes
// {l, l+16, l+32, l+48}, and the O^T accumulator rows match them.
// Within each 32-key MFMA step, lane group g feeds keys {4g..4g+3} and
// {16+4g..16+4g+3}; the V^T tile stores keys in that slot order so each A
// operand is one 16-byte LDS read.
//
// Pipeline: K/V tiles for block kb+1 are fetched into registers while block
// kb is computed from LDS (double buffered). Heavy (late) query blocks are
// scheduled first. An optional epilogue writes the chunk's K/V rows into the
// [Hkv, max_seq, D] cache (fused copy_to_cache).
#include "common.hpp"

#include <algorithm>
#include <atomic>

namespace aila {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr float kLazyRescaleLog2 = 8.0f;
constexpr int kPrefetch = 8;   // LDS operand reads in flight ahead of their MFMAs
constexpr int kNumXcd = 8;   // MI355X: 8 accelerator complex dies, one L2 each

template <int D, int RPW, int BN>
struct PrefillCfg {
  static constexpr int BM = kWaves * RPW;   // query rows of one 4-wave group
  static constexpr int QT = RPW / 16;     // 16-row query tiles per wave
  static constexpr int KS = D / 32;       // MFMA k-steps over D (S^T)
  static constexpr int DT = D / 16;       // 16-row d tiles (O^T)
  static constexpr int KT = BN / 16;      // 16-key tiles per block
  static constexpr int PS = BN / 32;      // 32-key MFMA steps (O^T)
  static constexpr int NC = D / 8;        // 16-byte chunks per K/V row
  static constexpr int RB = D * 2;        // bytes per K/V row
  static constexpr int TILE = BN * RB;    // one K or V tile (unpadded, swizzled)
  static constexpr int GROUP_BYTES = 4 * TILE;              // K, V x 2 buffers
  static constexpr int LOADS = BN * NC / kThreads;          // 16-byte DMA loads / thread / tile
  static constexpr int MERGE_HALF = kWaves * QT * (DT / 2) * 64 * 16;   // o_acc half, all waves
  static_assert(BN % 32 == 0 && D % 32 == 0 && RPW % 16 == 0, "tile");
  static_assert((BN * NC) % kThreads == 0, "whole DMA waves per tile");
  static_assert(MERGE_HALF <= 2 * TILE, "merge scratch fits in the buffer-0 K tiles");
  static_assert(kWaves * QT * 64 * 8 <= 2 * TILE, "m/l scratch fits in the buffer-0 V tiles");
};

// 16-byte chunk swizzles of the K and V tile rows (XOR on the chunk index).
// Tiles are written by DMA (one contiguous KiB per wave instruction, so rows
// cannot be padded). Measured on gfx950 over all bit-permutation swizzles of
// 256-byte rows: the S^T A-operand reads (ds_read_b128, 16 rows x one chunk
// per 16 lanes) reach ~245 B/clk/CU only when bit 0 of the swizzle comes from
// row bit 0 or 1 (else ~126), and the transposed V reads (ds_read_b64_tr_b16)
// reach ~166 B/clk/CU only when it comes from row bit 3 (else ~123). The two
// tiles are separate, so each gets its own.
template <int D>
__device__ __forceinline__ int swz_k(int r) {
  if constexpr (D >= 128) return r & 15;
  else return r & 7;                                 // 8 chunks per row
}
template <int D>
__device__ __forceinline__ int swz_v(int r) {
  if constexpr (D >= 128) return ((r & 7) << 1) | ((r >> 3) & 1);
  else return (((r >> 1) & 3) << 1) | ((r >> 3) & 1);
}

// One workgroup = two 4-wave groups and one head. It owns a balanced pair of
// query blocks: light block i and heavy block n-1-i (causal work grows with
// the block index, so every pair costs n+1 key blocks when start_pos = 0).
// Group A walks the light block's keys and then the first part of the heavy
// block's keys; group B walks the rest of the heavy block's keys; both walk
// the same number of key blocks (within one), each on its own double-buffered
// K/V tiles, and the heavy block's two partial softmax states are merged
// through LDS at the end.
//
// Schedule (ping-pong). A group alternates a matrix phase M(j) - O^T +=
// V_{j-1}^T P_{j-1}^T, then S_j^T = K_j Q^T - with a vector phase V(j) - the
// softmax of S_j into P_j. Group B runs one phase behind group A, with a
// workgroup barrier between phases, so on every SIMD one wave feeds the
// matrix core and reads LDS while the other runs the softmax on the vector
// ALU (the two overlap across waves, not within one wave).
//
// Tiles: M(j) reads K_j from Kbuf[j%2] and V_{j-1} from Vbuf[(j-1)%2]. When
// M(j) is done, V(j) refills exactly those two buffers by DMA with V_{j+1}
// and K_{j+2}, which M(j+1) and M(j+2) need three phases later; before
// M(j+1) each wave waits for its DMAs of V(j-1) only. The phase loop is
// unrolled by two so every LDS access names its buffer at compile time and
// the compiler can tell reads apart from the DMAs still in flight.
//
// K and V tiles are row-major [BN][D] in LDS (swizzled 16-byte chunks).
// O^T += V^T P^T takes its V^T operand from ds_read_b64_tr_b16: within a
// 16-lane group, lane i addresses 4 bf16 of row kbase + i/4 at column
// d0 + 4*(i%4), and lane j receives V[kbase+r][d0+j] for r = 0..3 - four
// keys of one head dim, the A-operand layout.
template <int D, int RPW, int BN, bool KSPLIT = false>
__global__ __launch_bounds__(2 * kThreads, 1) void gqa_prefill_kernel(
    const bf16* __restrict__ q, int q_row_stride, const bf16* __restrict__ k,
    const bf16* __restrict__ v, int kv_row_stride, long kv_head_stride,
    bf16* __restrict__ out, int o_row_stride, int S, int start_pos, int Hkv,
    int G, float scale_log2, bf16* __restrict__ k_cache,
    bf16* __restrict__ v_cache, int cache_pos, int max_seq, float* __restrict__ part) {
  using C = PrefillCfg<D, RPW, BN>;
  // K/V tiles per double-buffer slot, indexed by group.
  __shared__ __attribute__((aligned(1024))) unsigned char sK0[2][C::TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char sK1[2][C::TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char sV0[2][C::TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char sV1[2][C::TILE];
  // Group A's second (heavy) query block, staged by DMA in the prologue so
  // that switching blocks mid-loop costs LDS reads, not a memory round trip.
  __shared__ __attribute__((aligned(1024))) unsigned char sQh[kWaves * C::QT * C::KS * 1024];

  const int grp = __builtin_amdgcn_readfirstlane(threadIdx.x / kThreads);   // 0 = A, 1 = B
  const int t = threadIdx.x % kThreads, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int m16 = lane & 15, g4 = lane >> 4;

  const int nqb = (S + C::BM - 1) / C::BM;
  const int npair = (nqb + 1) / 2;
  // XCD-aware order: workgroups are dispatched round-robin over the 8 XCDs,
  // so consecutive logical ids (pairs of one head, then the heads of one KV
  // group) are gathered onto one XCD and its L2 holds that group's K/V.
  // With a key split (gridDim.z > 1, partial records in `part`), slice z of
  // the grid walks the z-th of gridDim.z equal runs of every query block's
  // key blocks; the slices of the same KV group and key run stay together.
  const int Hq = static_cast<int>(gridDim.y), nz = KSPLIT ? static_cast<int>(gridDim.z) : 1;
  const int nwg = npair * Hq * nz;
  const int lin = blockIdx.x + npair * (blockIdx.y + Hq * blockIdx.z);
  int logical = lin;
  if (nwg % kNumXcd == 0) logical = (lin % kNumXcd) * (nwg / kNumXcd) + lin / kNumXcd;
  const int pr = logical % npair;
  const int h = (logical / npair) % Hq;
  const int zs = KSPLIT ? logical / (npair * Hq) : 0;
  const int kvh = h / G;
  const int ql = pr, qh = nqb - 1 - pr;                  // light / heavy query block
  auto nkeyblk = [&](int qb) __attribute__((always_inline)) { return (start_pos + min((qb + 1) * C::BM, S) - 1) / BN + 1; };
  auto run_lo = [&](int qb) __attribute__((always_inline)) { return KSPLIT ? nkeyblk(qb) * zs / nz : 0; };
  auto run_hi = [&](int qb) __attribute__((always_inline)) {
    return KSPLIT ? nkeyblk(qb) * (zs + 1) / nz : nkeyblk(qb);
  };
  const int l0 = (ql < qh) ? run_lo(ql) : 0;
  const int nl = (ql < qh) ? run_hi(ql) - l0 : 0;       // a middle block pairs with itself
  const int h0 = run_lo(qh);
  const int nh = run_hi(qh) - h0;
  const int tA = (nl + nh + 1) / 2, tB = nl + nh - tA;   // tA >= tB
  const int hsplit = tA - nl;                           // heavy key blocks walked by A
  const int my_n = grp == 0 ? tA : tB;
  auto kb_of = [&](int it) __attribute__((always_inline)) {
    return grp == 0 ? (it < nl ? l0 + it : h0 + it - nl) : h0 + hsplit + it;
  };
  auto qb_of = [&](int it) __attribute__((always_inline)) { return (grp == 0 && it < nl) ? ql : qh; };
  const int kv_len = start_pos + S;
  const bf16* Kh = k + static_cast<size_t>(kvh) * kv_head_stride;
  const bf16* Vh = v + static_cast<size_t>(kvh) * kv_head_stride;

  // ---- K/V block -> LDS by DMA (wave-contiguous KiB per instruction) ------
  // Buffer loads straight into LDS. The buffer resource of a block starts at
  // its first key row and ends at its last row or the last valid row
  // (kv_len), whichever comes first, so rows past a ragged end read as zeros
  // (those keys are causally masked), every lane's byte offset is a constant
  // of the kernel, and the 32-bit range never spans more than one block.
  // (Fixed extent: an array sized by C::LOADS and captured by the lambdas
  // below makes the host pass drop the kernel's launch stub.)
  static_assert(C::LOADS <= 8, "dma_off extent");
  int koff[8], voff[8];
#pragma unroll
  for (int i = 0; i < C::LOADS; ++i) {
    const int p = (i * kWaves + wave) * 64 + lane;
    const int r = p / C::NC;
    koff[i] = (r * kv_row_stride + ((p % C::NC) ^ swz_k<D>(r)) * 8) * 2;
    voff[i] = (r * kv_row_stride + ((p % C::NC) ^ swz_v<D>(r)) * 8) * 2;
  }
  auto issue_tile = [&](unsigned char* tile, const bf16* base, const int* off, int kb) __attribute__((always_inline)) {
    const int key0 = kb * BN;
    const u32x4 src = buffer_rsrc(base + static_cast<size_t>(key0) * kv_row_stride,
                                  min(kv_len - key0, BN) * kv_row_stride * 2);
#pragma unroll
    for (int i = 0; i < C::LOADS; ++i) dma16_to_lds(src, off[i], tile + (i * kWaves + wave) * 64 * 16);
  };

  // ---- per-segment state ---------------------------------------------------
  bf16x8_t qb_op[C::QT][C::KS];
  f32x4 o_acc[C::DT][C::QT];
  float m_run[C::QT], l_run[C::QT];
  int seg_qb = -1;
  auto begin_segment = [&](int qb) __attribute__((always_inline)) {
    seg_qb = qb;
#pragma unroll
    for (int qt = 0; qt < C::QT; ++qt) {
      const int row = min(qb * C::BM + wave * RPW + qt * 16 + m16, S - 1);
      const bf16* qr = q + static_cast<size_t>(row) * q_row_stride + h * D + g4 * 8;
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks) qb_op[qt][ks] = as_bf16x8(ld16(qr + ks * 32));
      m_run[qt] = -INFINITY;
      l_run[qt] = 0.f;
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) o_acc[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  // The heavy block's Q operands of this wave, in [qt][ks][lane] order.
  unsigned char* my_qh = sQh + wave * (C::QT * C::KS * 1024);
  auto stage_segment_q = [&](int qb) __attribute__((always_inline)) {
    // a range over this block's rows only (rows past S clamp to the last)
    const int row0 = qb * C::BM;
    const u32x4 src = buffer_rsrc(q + static_cast<size_t>(row0) * q_row_stride + h * D,
                                  (min(row0 + C::BM, S) - 1 - row0) * q_row_stride * 2 + D * 2);
#pragma unroll
    for (int qt = 0; qt < C::QT; ++qt) {
      const int row = min(row0 + wave * RPW + qt * 16 + m16, S - 1) - row0;
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks)
        dma16_to_lds(src, (row * q_row_stride + g4 * 8 + ks * 32) * 2, my_qh + (qt * C::KS + ks) * 1024);
    }
  };
  auto begin_staged_segment = [&](int qb) __attribute__((always_inline)) {
    seg_qb = qb;
#pragma unroll
    for (int qt = 0; qt < C::QT; ++qt) {
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks)
        qb_op[qt][ks] = as_bf16x8(*reinterpret_cast<const u32x4*>(my_qh + (qt * C::KS + ks) * 1024 + lane * 16));
      m_run[qt] = -INFINITY;
      l_run[qt] = 0.f;
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) o_acc[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto store_segment = [&]() __attribute__((always_inline)) {
    if (KSPLIT) {
      // key split: the unnormalised state {m (log2 units), l, acc} of each
      // row, stride D + 4 floats, slice-major
#pragma unroll
      for (int qt = 0; qt < C::QT; ++qt) {
        const int row = seg_qb * C::BM + wave * RPW + qt * 16 + m16;
        if (row < S) {
          float* rec = part + ((static_cast<size_t>(zs) * Hq + h) * S + row) * (D + 4);
          if (g4 == 0) *reinterpret_cast<f32x4*>(rec) = f32x4{m_run[qt], l_run[qt], 0.f, 0.f};
#pragma unroll
          for (int dt = 0; dt < C::DT; ++dt)
            *reinterpret_cast<f32x4*>(rec + 4 + dt * 16 + g4 * 4) = o_acc[dt][qt];
        }
      }
      return;
    }
#pragma unroll
    for (int qt = 0; qt < C::QT; ++qt) {
      const float inv = 1.0f / l_run[qt];   // full row sum, held by every lane
      const int row = seg_qb * C::BM + wave * RPW + qt * 16 + m16;
      if (row < S) {
        bf16* orow = out + static_cast<size_t>(row) * o_row_stride + h * D + g4 * 4;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
          const f32x4 o = o_acc[dt][qt] * inv;
          const u32x2 w = {pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
          // outputs and cache rows are written once and not read back by
          // this kernel: nontemporal (config 2: 50.5 -> 48.5 us)
          __builtin_nontemporal_store(w, reinterpret_cast<u32x2*>(orow + dt * 16));
        }
      }
    }
  };

  // ---- S^T = K Q^T for one key block (matrix phase) -----------------------
  f32x4 st[C::KT][C::QT];
  bool s_valid = false, p_valid = false;
  int s_kb = 0;
  auto s_block = [&](const unsigned char* tk, int kb) __attribute__((always_inline)) {
    const int key0 = kb * BN;
    const int wave_qmin = start_pos + seg_qb * C::BM + wave * RPW;
    s_kb = kb;
    s_valid = key0 <= wave_qmin + RPW - 1;   // otherwise every key is in this wave's future
    if (!s_valid) return;
    // K operands in (ks, kt) order, each read kPrefetch operands ahead of the
    // MFMAs that use it; the schedule barriers keep that distance (left
    // alone, the scheduler issues each read just two MFMAs before its use).
    auto load_k = [&](int i) __attribute__((always_inline)) {
      const int ks = i / C::KT, kt = i % C::KT;
      const int r = kt * 16 + m16;
      return as_bf16x8(*reinterpret_cast<const u32x4*>(tk + r * C::RB + (((ks * 4 + g4) ^ swz_k<D>(r)) << 4)));
    };
#pragma unroll
    for (int kt = 0; kt < C::KT; ++kt)
#pragma unroll
      for (int qt = 0; qt < C::QT; ++qt) st[kt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    constexpr int NK = C::KS * C::KT;
    bf16x8_t kop[NK];
#pragma unroll
    for (int i = 0; i < kPrefetch && i < NK; ++i) kop[i] = load_k(i);
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      if (i + kPrefetch < NK) kop[i + kPrefetch] = load_k(i + kPrefetch);
      const int ks = i / C::KT, kt = i % C::KT;
#pragma unroll
      for (int qt = 0; qt < C::QT; ++qt) st[kt][qt] = mfma16x16x32(kop[i], qb_op[qt][ks], st[kt][qt]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // ---- softmax of S_j into P_j (vector phase) -------------------------------
  bf16x8_t pb[C::PS][C::QT];   // step s2 covers keys 32*s2 + {4g..4g+3, 16+4g..16+4g+3}
  auto softmax = [&](const bool masked) __attribute__((always_inline)) {
    const int key0 = s_kb * BN;
    const int wave_qmin = start_pos + seg_qb * C::BM + wave * RPW;
    if (masked) {
#pragma unroll
      for (int qt = 0; qt < C::QT; ++qt) {
        const int rel = wave_qmin + qt * 16 + m16 - key0 - g4 * 4;   // key offset limit
#pragma unroll
        for (int kt = 0; kt < C::KT; ++kt)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (kt * 16 + j > rel) st[kt][qt][j] = -INFINITY;
      }
    }
    // P at the running maxima, issued before the block's maxima are known;
    // the lazy rescale leaves a maximum in place unless the block exceeds it
    // by 2^8, so these are the final P of every row but where one grows (or
    // at a row's first block), when the wave recomputes its P below.
    auto exp_pass = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int qt = 0; qt < C::QT; ++qt) {
        const float nm = (m_run[qt] == -INFINITY) ? 0.f : -m_run[qt];
#pragma unroll
        for (int s2 = 0; s2 < C::PS; ++s2) {
          float p[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            p[j] = fast_exp2(fmaf(st[2 * s2][qt][j], scale_log2, nm));
            p[4 + j] = fast_exp2(fmaf(st[2 * s2 + 1][qt][j], scale_log2, nm));
          }
          const u32x4 w = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]),
                           pack_bf16x2(p[4], p[5]), pack_bf16x2(p[6], p[7])};
          pb[s2][qt] = as_bf16x8(w);
        }
      }
    };
    exp_pass();
    float alpha[C::QT];
    bool any_rescale = false;
#pragma unroll
    for (int qt = 0; qt < C::QT; ++qt) {
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < C::KT; ++kt)
#pragma unroll
        for (int j = 0; j < 4; ++j) mx = fmaxf(mx, st[kt][qt][j]);
      mx = xrow4_max(mx) * scale_log2;
      const bool grow = mx > m_run[qt] + kLazyRescaleLog2;
      const float mn = grow ? mx : m_run[qt];
      alpha[qt] = grow ? ((m_run[qt] == -INFINITY) ? 0.f : fast_exp2(m_run[qt] - mn)) : 1.0f;
      m_run[qt] = mn;
      any_rescale |= grow;
    }
    // o_acc and l hold every block before j (M(j) added P_{j-1}).
    if (__any(any_rescale)) {
      exp_pass();
#pragma unroll
      for (int qt = 0; qt < C::QT; ++qt) {
        l_run[qt] *= alpha[qt];
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) o_acc[dt][qt] *= alpha[qt];
      }
    }
  };

  // ---- O^T += V^T P^T and l += rowsum(P) (matrix phase) ---------------------
  auto pv_block = [&](const unsigned char* tv) __attribute__((always_inline)) {
    // V^T operands come from transposing LDS reads, in (s2, dt) order, each
    // read kPrefetch operands ahead of its MFMAs (as the K operands above).
    const int vr = 4 * g4 + (m16 >> 2);          // row within a 32-key step (first half)
    const int vc = 4 * (m16 & 3);                // column offset within a 16-wide d tile
    auto load_v = [&](int i) __attribute__((always_inline)) {
      const int s2 = i / C::DT, dt = i % C::DT;
      const int d = dt * 16 + vc;
      const int r0 = s2 * 32 + vr, r1 = r0 + 16;
      const unsigned char* p0 = tv + r0 * C::RB + (((d >> 3) ^ swz_v<D>(r0)) << 4) + ((d & 7) << 1);
      const unsigned char* p1 = tv + r1 * C::RB + (((d >> 3) ^ swz_v<D>(r1)) << 4) + ((d & 7) << 1);
      const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)p0);
      const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)p1);
      const u32x4 w = {__builtin_bit_cast(u32x2, lo)[0], __builtin_bit_cast(u32x2, lo)[1],
                       __builtin_bit_cast(u32x2, hi)[0], __builtin_bit_cast(u32x2, hi)[1]};
      return as_bf16x8(w);
    };
    constexpr int NV = C::PS * C::DT;
    bf16x8_t vop[NV];
#pragma unroll
    for (int i = 0; i < kPrefetch && i < NV; ++i) vop[i] = load_v(i);
    // Row sums of P on the matrix cores while the first reads are in flight:
    // a ones A operand gives every output row the column sums of P^T, i.e.
    // the full row sum of each query (all 32 keys of the step, the bf16 P the
    // numerator uses) in every lane.
    {
      const u32x4 ones_w = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
      const bf16x8_t ones = as_bf16x8(ones_w);
#pragma unroll
      for (int qt = 0; qt < C::QT; ++qt) {
        f32x4 ls = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s2 = 0; s2 < C::PS; ++s2) ls = mfma16x16x32(ones, pb[s2][qt], ls);
        l_run[qt] += ls[0];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (i + kPrefetch < NV) vop[i + kPrefetch] = load_v(i + kPrefetch);
      const int s2 = i / C::DT, dt = i % C::DT;
#pragma unroll
      for (int qt = 0; qt < C::QT; ++qt) o_acc[dt][qt] = mfma16x16x32(vop[i], pb[s2][qt], o_acc[dt][qt]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // ---- fused copy_to_cache: this pair's own K/V rows, shared by the G query
  //      heads of the KV group (head h copies every G-th row from h % G).
  auto copy_rows_to_cache = [&](int tid0, int nthr) __attribute__((always_inline)) {
    if (k_cache != nullptr) {
      const int gi = h % G;
#pragma unroll 1
      for (int pass = 0; pass < 2; ++pass) {
        const int qb = pass == 0 ? qh : ql;
        if (pass == 1 && ql == qh) break;
        const int r0 = qb * C::BM, r1 = min(r0 + C::BM, S);
        const int nrow = (r1 - r0 - gi + G - 1) / G;   // rows r0 + gi, r0 + gi + G, ...
        for (int p = tid0; p < nrow * C::NC; p += nthr) {
          const int row = r0 + gi + (p / C::NC) * G, c = p % C::NC;
          const size_t src = static_cast<size_t>(row) * kv_row_stride + c * 8;
          const size_t dst = (static_cast<size_t>(kvh) * max_seq + cache_pos + row) * D + c * 8;
          __builtin_nontemporal_store(ld16(Kh + src), reinterpret_cast<u32x4*>(k_cache + dst));
          __builtin_nontemporal_store(ld16(Vh + src), reinterpret_cast<u32x4*>(v_cache + dst));
        }
      }
    }
  };

  // ---- prologue: K_0, V_0, K_1 (+ group A's heavy Q) ------------------------
  if (my_n > 0) {
    begin_segment(qb_of(0));
    issue_tile(sK0[grp], Kh, koff, kb_of(0));
    issue_tile(sV0[grp], Vh, voff, kb_of(0));
    if (my_n > 1) issue_tile(sK1[grp], Kh, koff, kb_of(1));
    if (grp == 0 && nl > 0 && hsplit > 0) stage_segment_q(qh);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm<0>());
  __syncthreads();

  // One block step: matrix phase M(j), barrier, vector phase V(j), barrier.
  // The phase barriers fence LDS only: inside the loop LDS is written only by
  // the DMAs, whose completion the explicit vmcnt waits establish (a full
  // __syncthreads would wait for every DMA still in flight).
  // kcur = Kbuf[j%2] (K_j, then refilled with K_{j+2}); vprev = Vbuf[(j+1)%2]
  // (V_{j-1}, then refilled with V_{j+1}).
  const int nsteps = tA;   // both groups run tA steps; B's last is empty when tB < tA
  auto step = [&](int j, unsigned char* kcur, unsigned char* vprev) __attribute__((always_inline)) {
    // M(j)
    if (j >= 1 && j - 1 < my_n && p_valid) pv_block(vprev);
    if (j < my_n) {
      if (j >= 1 && qb_of(j) != qb_of(j - 1)) {   // group A moves from its light to its heavy block
        store_segment();
        begin_staged_segment(qb_of(j));             // staged in the prologue, long complete
      }
      s_block(kcur, kb_of(j));
    } else {
      s_valid = false;
    }
    phase_barrier();
    if (j >= nsteps) return;
    // V(j)
    const bool nv = j + 1 < my_n, nk = j + 2 < my_n;
    if (nv) issue_tile(vprev, Vh, voff, kb_of(j + 1));
    if (nk) issue_tile(kcur, Kh, koff, kb_of(j + 2));
    p_valid = s_valid;
    if (s_valid) {
      if (s_kb * BN + BN - 1 > start_pos + seg_qb * C::BM + wave * RPW) softmax(true);
      else softmax(false);
    }
    // M(j+1) needs K_{j+1} and V_j, issued in V(j-1): only this phase's DMAs
    // may stay in flight.
    if (nk) __builtin_amdgcn_s_waitcnt(vmcnt_imm<2 * C::LOADS>());
    else if (nv) __builtin_amdgcn_s_waitcnt(vmcnt_imm<C::LOADS>());
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm<0>());
    phase_barrier();
  };
  if (grp == 1) phase_barrier();   // group B runs one phase behind
  for (int j = 0; j <= nsteps; j += 2) {
    step(j, sK0[grp], sV1[grp]);
    if (j + 1 <= nsteps) step(j + 1, sK1[grp], sV0[grp]);
  }
  // Group A copies the pair's K/V rows to the cache while group B runs its
  // last matrix phase (config 2: 43.7 -> 43.3 us against all 512 threads
  // copying after the merge).
  if (grp == 0) {
    copy_rows_to_cache(t, kThreads);
    phase_barrier();
  }

  // ---- finish: light block of A, heavy block (merged when split) -------------
  __builtin_amdgcn_s_waitcnt(vmcnt_imm<0>());
  __syncthreads();
  const bool a_has_heavy = hsplit > 0;
  const bool b_has_heavy = tB > 0;
  if (grp == 0 && !a_has_heavy && nl > 0) store_segment();          // A only had the light block
  if (a_has_heavy && b_has_heavy) {
    // A publishes its heavy partial state; B merges and stores. The o_acc
    // exchange goes in two halves of the d tiles through the buffer-0 K
    // tiles; m and l through the buffer-0 V tiles.
    float* o_scr = reinterpret_cast<float*>(&sK0[0][0]) + wave * (C::QT * (C::DT / 2) * 64 * 4);
    float* ml_scr = reinterpret_cast<float*>(&sV0[0][0]) + wave * (C::QT * 64 * 2);
    float fa[C::QT], fb[C::QT];
    if (grp == 0) {
#pragma unroll
      for (int qt = 0; qt < C::QT; ++qt) {
        ml_scr[(qt * 64 + lane) * 2] = m_run[qt];
        ml_scr[(qt * 64 + lane) * 2 + 1] = l_run[qt];
      }
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      if (grp == 0) {
#pragma unroll
        for (int qt = 0; qt < C::QT; ++qt)
#pragma unroll
          for (int dd = 0; dd < C::DT / 2; ++dd)
            *reinterpret_cast<f32x4*>(&o_scr[((qt * (C::DT / 2) + dd) * 64 + lane) * 4]) = o_acc[half * (C::DT / 2) + dd][qt];
      }
      __syncthreads();
      if (grp == 1) {
#pragma unroll
        for (int qt = 0; qt < C::QT; ++qt) {
          if (half == 0) {
            const float ma = ml_scr[(qt * 64 + lane) * 2], la = ml_scr[(qt * 64 + lane) * 2 + 1];
            const float M = fmaxf(ma, m_run[qt]);
            fa[qt] = (ma == -INFINITY) ? 0.f : fast_exp2(ma - M);
            fb[qt] = (m_run[qt] == -INFINITY) ? 0.f : fast_exp2(m_run[qt] - M);
            l_run[qt] = fa[qt] * la + fb[qt] * l_run[qt];
            m_run[qt] = M;   // l and acc are now relative to M (a key-split record carries it)
          }
#pragma unroll
          for (int dd = 0; dd < C::DT / 2; ++dd) {
            const int dt = half * (C::DT / 2) + dd;
            o_acc[dt][qt] = fa[qt] * *reinterpret_cast<const f32x4*>(&o_scr[((qt * (C::DT / 2) + dd) * 64 + lane) * 4]) +
                            fb[qt] * o_acc[dt][qt];
          }
        }
      }
      __syncthreads();
    }
    if (grp == 1) store_segment();
  } else if (a_has_heavy && grp == 0) {
    store_segment();
  } else if (b_has_heavy && grp == 1) {
    store_segment();
  }
}

// Key-split merge: out row = sum_z 2^(m_z - M) acc_z / sum_z 2^(m_z - M) l_z
// over the slices' partial records (M = max m_z; a slice whose keys were
// all masked for the row has m = -inf and weight 0). D/4 threads per
// (row, head), one float4 column each.
template <int D>
__global__ __launch_bounds__(256) void gqa_prefill_merge_kernel(const float* __restrict__ part,
                                                                bf16* __restrict__ out, int o_row_stride, int S,
                                                                int Hq, int nz) {
  constexpr int TPR = D / 4;
  constexpr int RPB = 256 / TPR;
  const long idx = static_cast<long>(blockIdx.x) * RPB + threadIdx.x / TPR;   // row * Hq + h
  if (idx >= static_cast<long>(S) * Hq) return;
  const int row = static_cast<int>(idx / Hq), h = static_cast<int>(idx % Hq), c = (threadIdx.x % TPR) * 4;
  const size_t slice = static_cast<size_t>(Hq) * S * (D + 4);
  const float* rec = part + (static_cast<size_t>(h) * S + row) * (D + 4);
  float M = -INFINITY;
  for (int z = 0; z < nz; ++z) M = fmaxf(M, rec[z * slice]);
  float L = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int z = 0; z < nz; ++z) {
    const float m = rec[z * slice];
    const float w = (m == -INFINITY) ? 0.f : fast_exp2(m - M);
    L += w * rec[z * slice + 1];
    acc += w * *reinterpret_cast<const f32x4*>(rec + z * slice + 4 + c);
  }
  // Every run of every row is non-empty (the host caps nz at the first query
  // block's key-block count, so run z of n >= nz blocks holds
  // floor(n(z+1)/nz) - floor(nz z/nz) >= 1 blocks, and each row's diagonal
  // key lies in some run): every record is written and L > 0. The guard
  // keeps a zero row instead of NaN should that ever break.
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  *reinterpret_cast<u32x2*>(out + static_cast<size_t>(row) * o_row_stride + h * D + c) =
      u32x2{pack_bf16x2(acc[0] * inv, acc[1] * inv), pack_bf16x2(acc[2] * inv, acc[3] * inv)};
}

template <int D, int RPW, int BN>
int launch_prefill(const bf16* q, const bf16* k, const bf16* v, int kv_row_stride,
                   long kv_head_stride, bf16* out, int S, int start_pos, int Hq,
                   int Hkv, bf16* k_cache, bf16* v_cache, int cache_pos, int max_seq,
                   int nz, float* part, hipStream_t st) {
  using C = PrefillCfg<D, RPW, BN>;
  const int nqb = (S + C::BM - 1) / C::BM;
  const int npair = (nqb + 1) / 2;
  const float scale_log2 = kLog2e / sqrtf(static_cast<float>(D));
  // Each key run must hold at least one key block of every query block, so
  // that every record the merge reads is written: the first query block has
  // the fewest key blocks.
  const int min_blocks = (start_pos + (S < C::BM ? S : C::BM) - 1) / BN + 1;
  if (nz > min_blocks) nz = min_blocks;
  if (nz < 2) {
    nz = 1;
    part = nullptr;
  }
  if (part == nullptr)
    hipLaunchKernelGGL((gqa_prefill_kernel<D, RPW, BN, false>), dim3(npair, Hq), dim3(2 * kThreads), 0, st,
                       q, Hq * D, k, v, kv_row_stride, kv_head_stride, out, Hq * D, S, start_pos,
                       Hkv, Hq / Hkv, scale_log2, k_cache, v_cache, cache_pos, max_seq, nullptr);
  else
    hipLaunchKernelGGL((gqa_prefill_kernel<D, RPW, BN, true>), dim3(npair, Hq, nz), dim3(2 * kThreads), 0, st,
                       q, Hq * D, k, v, kv_row_stride, kv_head_stride, out, Hq * D, S, start_pos,
                       Hkv, Hq / Hkv, scale_log2, nullptr, nullptr, 0, max_seq, part);
  if (part != nullptr) {
    constexpr int RPB = 256 / (D / 4);
    const long rows = static_cast<long>(S) * Hq;
    hipLaunchKernelGGL((gqa_prefill_merge_kernel<D>), dim3(static_cast<unsigned>((rows + RPB - 1) / RPB)),
                       dim3(256), 0, st, part, out, Hq * D, S, Hq, nz);
  }
  return check_launch("gqa_prefill");
}

template <int D>
struct PrefillShape;
template <>
struct PrefillShape<64> { static constexpr int RPW = 32, BN = 64; };
template <>
struct PrefillShape<128> { static constexpr int RPW = 32, BN = 64; };
template <>
struct PrefillShape<256> { static constexpr int RPW = 16, BN = 32; };

// Prefill workgroups the device holds at once, per device (idempotent,
// computed on first use).
template <int D>
int prefill_resident() {
  using PS = PrefillShape<D>;
  constexpr int kMaxDev = 64;
  static std::atomic<int> cache[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 256;
  const int known = cache[dev].load(std::memory_order_relaxed);
  if (known > 0) return known;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gqa_prefill_kernel<D, PS::RPW, PS::BN, true>, 2 * kThreads,
                                                   0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu <= 0 ||
      cus <= 0)
    return 256;
  cache[dev].store(per_cu * cus, std::memory_order_relaxed);
  return per_cu * cus;
}

constexpr int kMaxKeySplits = 16;

// Key runs per query block for a prefill over a cached prefix: enough
// workgroups for one round of the device, each run at least 4 key blocks
// long (the short runs' per-workgroup start-up would cost more than they
// save). 1 = no split.
template <int D>
int prefill_key_splits(int S, int start_pos, int Hq) {
  using PS = PrefillShape<D>;
  using C = PrefillCfg<D, PS::RPW, PS::BN>;
  const int nqb = (S + C::BM - 1) / C::BM;
  const int nwg = (nqb + 1) / 2 * Hq;
  const int resident = prefill_resident<D>();
  if (2 * nwg > resident) return 1;
  const int min_blocks = (start_pos + std::min(C::BM, S) - 1) / PS::BN + 1;   // the first query block's keys
  int nz = (resident + nwg - 1) / nwg;
  // at least 4 key blocks per run; launch_prefill relies on >= 1
  nz = std::min(nz, std::min(kMaxKeySplits, min_blocks / 4));
  return nz < 2 ? 1 : nz;
}

int key_splits_for(int D, int S, int start_pos, int Hq) {
  switch (D) {
    case 64: return prefill_key_splits<64>(S, start_pos, Hq);
    case 128: return prefill_key_splits<128>(S, start_pos, Hq);
    case 256: return prefill_key_splits<256>(S, start_pos, Hq);
    default: return 1;
  }
}

size_t key_split_bytes(int nz, int S, int Hq, int D) {
  return static_cast<size_t>(nz) * Hq * S * (D + 4) * sizeof(float);
}

// Short sequences and few heads leave most CUs idle with 32 query rows per
// wave (one workgroup per balanced pair of 128-row blocks and head). When
// 16 rows per wave (64-row blocks, twice the workgroups, twice the LDS
// operand bytes per MFMA) still fits one round of the device, it is faster
// (Hq=32, Hkv=8, D=128: S=512 20.4 -> 13.5 us, S=1024 28.5 -> 20.8;
// Hq=8, Hkv=2, S=4096 65.4 -> 47.5); two rounds are slower (S=1280: 32.0
// against 40.2), so larger grids keep 32 rows per wave. So does a
// sequence that gets no more workgroups from it (S = 65..128: one pair
// either way, and over a 4096-row cached prefix 81 against 64 us), unless
// the 128-row block would be half padding (S <= 64: 61 -> 43 us over the
// same prefix).
template <int D>
bool short_prefill(int S, int Hq, int nz) {
  if (nz > 1) return false;
  const long npair16 = ((S + 63) / 64 + 1) / 2;
  const long npair32 = ((S + 127) / 128 + 1) / 2;
  return (npair16 > npair32 || S <= 64) && npair16 * Hq <= prefill_resident<D>();
}

int dispatch_prefill(int D, const bf16* q, const bf16* k, const bf16* v, int kv_row_stride,
                     long kv_head_stride, bf16* out, int S, int start_pos, int Hq, int Hkv,
                     bf16* k_cache, bf16* v_cache, int cache_pos, int max_seq, hipStream_t st,
                     int nz = 1, float* part = nullptr) {
  switch (D) {
    case 64:
      if (short_prefill<64>(S, Hq, nz))
        return launch_prefill<64, 16, 64>(q, k, v, kv_row_stride, kv_head_stride, out, S, start_pos, Hq, Hkv, k_cache,
                                          v_cache, cache_pos, max_seq, nz, part, st);
      return launch_prefill<64, PrefillShape<64>::RPW, PrefillShape<64>::BN>(
          q, k, v, kv_row_stride, kv_head_stride, out, S, start_pos, Hq, Hkv, k_cache, v_cache, cache_pos, max_seq,
          nz, part, st);
    case 128:
      if (short_prefill<128>(S, Hq, nz))
        return launch_prefill<128, 16, 64>(q, k, v, kv_row_stride, kv_head_stride, out, S, start_pos, Hq, Hkv, k_cache,
                                           v_cache, cache_pos, max_seq, nz, part, st);
      return launch_prefill<128, PrefillShape<128>::RPW, PrefillShape<128>::BN>(
          q, k, v, kv_row_stride, kv_head_stride, out, S, start_pos, Hq, Hkv, k_cache, v_cache, cache_pos, max_seq,
          nz, part, st);
    case 256:
      return launch_prefill<256, PrefillShape<256>::RPW, PrefillShape<256>::BN>(
          q, k, v, kv_row_stride, kv_head_stride, out, S, start_pos, Hq, Hkv, k_cache, v_cache, cache_pos, max_seq,
          nz, part, st);
    default:
      return set_error(AILA_HIP_EUNSUPPORTED, "gqa_prefill: D=%d not in {64,128,256}", D);
  }
}

// copy_to_cache, AttentionOps.cpp:2513-2532: [S, H*D] -> [H, max_seq, D].
__global__ void copy_to_cache_kernel(const u32x4* __restrict__ src, bf16* __restrict__ cache,
                                     int S, int start_pos, int H, int D, int max_seq) {
  const int chunks = H * D / 8;
  const long n = static_cast<long>(S) * chunks;
  for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<long>(gridDim.x) * blockDim.x) {
    const int s = static_cast<int>(i / chunks), c = static_cast<int>(i % chunks);
    const int hh = (c * 8) / D, d = (c * 8) % D;
    *reinterpret_cast<u32x4*>(cache + (static_cast<size_t>(hh) * max_seq + start_pos + s) * D + d) = src[i];
  }
}

}  // namespace
}  // namespace aila

extern "C" int aila_hip_gqa_prefill(const void* q, const void* k, const void* v, void* out,
                                    void* k_cache, void* v_cache, int cache_pos, int max_seq,
                                    int S, int Hq, int Hkv, int D, void* stream) {
  using namespace aila;
  AILA_REQUIRE(q && k && v && out, "gqa_prefill: null pointer");
  AILA_REQUIRE(S > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq <= 65535,
               "gqa_prefill: bad shape (S=%d Hq=%d Hkv=%d)", S, Hq, Hkv);
  AILA_REQUIRE((k_cache == nullptr) == (v_cache == nullptr), "gqa_prefill: pass both caches or neither");
  if (k_cache) {
    AILA_REQUIRE(cache_pos >= 0 && static_cast<long>(cache_pos) + S <= max_seq,
                 "gqa_prefill: cache rows [%d, %d) exceed max_seq=%d", cache_pos, cache_pos + S, max_seq);
  }
  return dispatch_prefill(D, static_cast<const bf16*>(q), static_cast<const bf16*>(k),
                          static_cast<const bf16*>(v), Hkv * D, D, static_cast<bf16*>(out), S, 0, Hq,
                          Hkv, static_cast<bf16*>(k_cache), static_cast<bf16*>(v_cache), cache_pos,
                          max_seq, static_cast<hipStream_t>(stream));
}

extern "C" size_t aila_hip_gqa_prefill_cached_workspace_size(int S, int start_pos, int Hq, int Hkv, int D) {
  using namespace aila;
  if (S <= 0 || start_pos < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || (D != 64 && D != 128 && D != 256)) return 0;
  const int nz = key_splits_for(D, S, start_pos, Hq);
  return nz > 1 ? key_split_bytes(nz, S, Hq, D) : 0;
}

extern "C" int aila_hip_gqa_prefill_cached_ws(const void* q, const void* k_cache, const void* v_cache, void* out,
                                              void* workspace, size_t workspace_bytes, int S, int start_pos,
                                              int Hq, int Hkv, int D, int max_seq, void* stream) {
  using namespace aila;
  AILA_REQUIRE(q && k_cache && v_cache && out, "gqa_prefill_cached: null pointer");
  AILA_REQUIRE(S > 0 && start_pos >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq <= 65535,
               "gqa_prefill_cached: bad shape (S=%d start_pos=%d Hq=%d Hkv=%d)", S, start_pos, Hq, Hkv);
  AILA_REQUIRE(static_cast<long>(start_pos) + S <= max_seq,
               "gqa_prefill_cached: start_pos + S = %ld > max_seq=%d", static_cast<long>(start_pos) + S, max_seq);
  // a cache head's extent (max_seq * D) is passed to the kernel as an int
  AILA_REQUIRE(static_cast<long>(max_seq) * D * 2 < (1L << 31),
               "gqa_prefill_cached: a cache head (max_seq=%d, D=%d) exceeds 2 GiB", max_seq, D);
  AILA_REQUIRE(workspace == nullptr || reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
               "gqa_prefill_cached: workspace not 16-byte aligned");
  int nz = 1;
  if (workspace != nullptr && (D == 64 || D == 128 || D == 256)) {
    nz = key_splits_for(D, S, start_pos, Hq);
    // as many key runs as the workspace holds
    const size_t per = key_split_bytes(1, S, Hq, D);
    nz = static_cast<int>(std::min<size_t>(static_cast<size_t>(nz), workspace_bytes / per));
  }
  return dispatch_prefill(D, static_cast<const bf16*>(q), static_cast<const bf16*>(k_cache),
                          static_cast<const bf16*>(v_cache), D, static_cast<long>(max_seq) * D,
                          static_cast<bf16*>(out), S, start_pos, Hq, Hkv, nullptr, nullptr, 0, max_seq,
                          static_cast<hipStream_t>(stream), nz, static_cast<float*>(workspace));
}

extern "C" int aila_hip_gqa_prefill_cached(const void* q, const void* k_cache, const void* v_cache,
                                           void* out, int S, int start_pos, int Hq, int Hkv, int D,
                                           int max_seq, void* stream) {
  return aila_hip_gqa_prefill_cached_ws(q, k_cache, v_cache, out, nullptr, 0, S, start_pos, Hq, Hkv, D, max_seq,
                                        stream);
}

extern "C" int aila_hip_copy_to_cache(const void* new_kv, void* cache, int S, int start_pos, int H,
                                      int D, int max_seq, void* stream) {
  using namespace aila;
  AILA_REQUIRE(new_kv && cache, "copy_to_cache: null pointer");
  AILA_REQUIRE(S >= 0 && H > 0 && D > 0 && D % 8 == 0, "copy_to_cache: bad shape (S=%d H=%d D=%d)", S, H, D);
  AILA_REQUIRE(start_pos >= 0 && static_cast<long>(start_pos) + S <= max_seq,
               "copy_to_cache: rows [%d, %d) exceed max_seq=%d", start_pos, start_pos + S, max_seq);
  if (S == 0) return AILA_HIP_OK;
  const long n = static_cast<long>(S) * H * D / 8;
  const int blocks = static_cast<int>(std::min<long>((n + 255) / 256, 4096));
  hipLaunchKernelGGL(copy_to_cache_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(new_kv), static_cast<bf16*>(cache), S, start_pos, H, D, max_seq);
  return check_launch("copy_to_cache");
}

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

namespace aila {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr float kLazyRescaleLog2 = 8.0f;
constexpr int kNumXcd = 8;   // MI355X: 8 accelerator complex dies, one L2 each
// s_waitcnt immediate (gfx9 encoding): vmcnt = 0, expcnt and lgkmcnt not waited on.
constexpr int kWaitVmcntZero = 0x0F70;

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

// 16-byte chunk swizzle of K/V tile rows. Tiles are written by direct
// global->LDS loads (one contiguous KiB per wave instruction, so rows cannot
// be padded); the XOR keeps both read patterns conflict-free: the S^T A
// operand (16 rows x one 16-byte chunk) and the transposed V reads (8 rows x
// one 32-byte chunk pair per half wave).
template <int D>
__device__ __forceinline__ int swz(int r) {
  if constexpr (D >= 128) return ((r & 7) << 1) | ((r >> 3) & 1);
  else return (((r >> 1) & 3) << 1) | ((r >> 3) & 1);        // 8 chunks per row
}

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16_t;

// One workgroup = two 4-wave groups and one head. It owns a balanced pair of
// query blocks: light block i and heavy block n-1-i (causal work grows with
// the block index, so every pair costs n+1 key blocks when start_pos = 0).
// Group A walks the light block's keys and then the first part of the heavy
// block's keys; group B walks the rest of the heavy block's keys; both run
// the same number of iterations (within one), each on its own double-buffered
// K/V tiles, and the heavy block's two partial softmax states are merged
// through LDS at the end.
//
// K and V tiles are row-major [BN][D] in LDS, filled by global_load_lds
// (no staging registers). O^T += V^T P^T takes its V^T operand from
// ds_read_b64_tr_b16: within a 16-lane group, lane i addresses 4 bf16 of
// row kbase + i/4 at column d0 + 4*(i%4), and lane j receives V[kbase+r][d0+j]
// for r = 0..3 - four keys of one head dim, the A-operand layout.
template <int D, int RPW, int BN>
__global__ __launch_bounds__(2 * kThreads, 1) void gqa_prefill_kernel(
    const bf16* __restrict__ q, int q_row_stride, const bf16* __restrict__ k,
    const bf16* __restrict__ v, int kv_row_stride, long kv_head_stride,
    bf16* __restrict__ out, int o_row_stride, int S, int start_pos, int Hkv,
    int G, float scale_log2, bf16* __restrict__ k_cache,
    bf16* __restrict__ v_cache, int cache_pos, int max_seq) {
  using C = PrefillCfg<D, RPW, BN>;
  // K/V tiles per double-buffer slot, indexed by group.
  __shared__ __attribute__((aligned(1024))) unsigned char sK0[2][C::TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char sK1[2][C::TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char sV0[2][C::TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char sV1[2][C::TILE];

  const int grp = __builtin_amdgcn_readfirstlane(threadIdx.x / kThreads);   // 0 = A, 1 = B
  const int t = threadIdx.x % kThreads, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int m16 = lane & 15, g4 = lane >> 4;
  auto tileK = [&](int buf) __attribute__((always_inline)) -> unsigned char* { return buf ? sK1[grp] : sK0[grp]; };
  auto tileV = [&](int buf) __attribute__((always_inline)) -> unsigned char* { return buf ? sV1[grp] : sV0[grp]; };

  const int nqb = (S + C::BM - 1) / C::BM;
  const int npair = (nqb + 1) / 2;
  // XCD-aware order: workgroups are dispatched round-robin over the 8 XCDs,
  // so consecutive logical ids (pairs of one head, then the heads of one KV
  // group) are gathered onto one XCD and its L2 holds that group's K/V.
  const int nwg = npair * static_cast<int>(gridDim.y);
  const int lin = blockIdx.x + npair * blockIdx.y;
  int logical = lin;
  if (nwg % kNumXcd == 0) logical = (lin % kNumXcd) * (nwg / kNumXcd) + lin / kNumXcd;
  const int pr = logical % npair;
  const int h = logical / npair;
  const int kvh = h / G;
  const int ql = pr, qh = nqb - 1 - pr;                  // light / heavy query block
  auto nkeyblk = [&](int qb) __attribute__((always_inline)) { return (start_pos + min((qb + 1) * C::BM, S) - 1) / BN + 1; };
  const int nl = (ql < qh) ? nkeyblk(ql) : 0;           // a middle block pairs with itself
  const int nh = nkeyblk(qh);
  const int tA = (nl + nh + 1) / 2, tB = nl + nh - tA;
  const int hsplit = tA - nl;                           // heavy key blocks walked by A
  const int my_n = grp == 0 ? tA : tB;
  auto kb_of = [&](int it) __attribute__((always_inline)) { return grp == 0 ? (it < nl ? it : it - nl) : hsplit + it; };
  auto qb_of = [&](int it) __attribute__((always_inline)) { return (grp == 0 && it < nl) ? ql : qh; };
  const int kv_len = start_pos + S;
  const bf16* Kh = k + kvh * kv_head_stride;
  const bf16* Vh = v + kvh * kv_head_stride;
  const bool cache_head = (k_cache != nullptr) && (h % G == 0);

  // ---- K/V block -> LDS by DMA (wave-contiguous KiB per instruction) ------
  // Per-lane element offsets of the DMA sources relative to the block's first
  // key row, fixed for the whole kernel; a block then only adds a uniform
  // base. The last block of a ragged length clamps its rows instead.
  // (Fixed extent: an array sized by C::LOADS and captured by the lambdas
  // below makes the host pass drop the kernel's launch stub.)
  static_assert(C::LOADS <= 8, "dma_off extent");
  int dma_off[8];
#pragma unroll
  for (int i = 0; i < C::LOADS; ++i) {
    const int p = (i * kWaves + wave) * 64 + lane;
    const int r = p / C::NC, qc = (p % C::NC) ^ swz<D>(r);
    dma_off[i] = r * kv_row_stride + qc * 8;
  }
  auto issue = [&](int buf, int kb) __attribute__((always_inline)) {
    const int key0 = kb * BN;
    unsigned char* tk = tileK(buf);
    unsigned char* tv = tileV(buf);
    if (key0 + BN <= kv_len) {
      const bf16* kb0 = Kh + static_cast<size_t>(key0) * kv_row_stride;
      const bf16* vb0 = Vh + static_cast<size_t>(key0) * kv_row_stride;
#pragma unroll
      for (int i = 0; i < C::LOADS; ++i) {
        const int wchunk = (i * kWaves + wave) * 64;
        __builtin_amdgcn_global_load_lds(kb0 + dma_off[i], (lds_void_t*)(tk + wchunk * 16), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vb0 + dma_off[i], (lds_void_t*)(tv + wchunk * 16), 16, 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < C::LOADS; ++i) {
        const int wchunk = (i * kWaves + wave) * 64;     // first 16-byte slot of this wave instruction
        const int p = wchunk + lane;
        const int r = p / C::NC, qc = (p % C::NC) ^ swz<D>(r);
        const size_t goff = static_cast<size_t>(min(key0 + r, kv_len - 1)) * kv_row_stride + qc * 8;
        __builtin_amdgcn_global_load_lds(Kh + goff, (lds_void_t*)(tk + wchunk * 16), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(Vh + goff, (lds_void_t*)(tv + wchunk * 16), 16, 0, 0);
      }
    }
  };
  // The chunk's own key rows of query block qb go to the cache (fused
  // copy_to_cache), copied out of the LDS tiles.
  auto write_cache = [&](int buf, int kb, int qb) __attribute__((always_inline)) {
    const int key0 = kb * BN;
    const int cq0 = qb * C::BM, cq1 = min(cq0 + C::BM, S) - 1;
    if (!(cache_head && key0 + BN - 1 >= cq0 && key0 <= cq1)) return;
    const unsigned char* tk = tileK(buf);
    const unsigned char* tv = tileV(buf);
#pragma unroll
    for (int i = 0; i < C::LOADS; ++i) {
      const int p = i * kThreads + t;
      const int r = p / C::NC, qc = (p % C::NC) ^ swz<D>(r);
      const int key = key0 + r;
      if (key >= cq0 && key <= cq1) {
        const size_t dst = (static_cast<size_t>(kvh) * max_seq + cache_pos + key) * D + qc * 8;
        *reinterpret_cast<u32x4*>(k_cache + dst) = *reinterpret_cast<const u32x4*>(tk + p * 16);
        *reinterpret_cast<u32x4*>(v_cache + dst) = *reinterpret_cast<const u32x4*>(tv + p * 16);
      }
    }
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
  auto store_segment = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int qt = 0; qt < C::QT; ++qt) {
      float l = l_run[qt];
      l += __shfl_xor(l, 16);
      l += __shfl_xor(l, 32);
      const float inv = 1.0f / l;
      const int row = seg_qb * C::BM + wave * RPW + qt * 16 + m16;
      if (row < S) {
        bf16* orow = out + static_cast<size_t>(row) * o_row_stride + h * D + g4 * 4;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
          const f32x4 o = o_acc[dt][qt] * inv;
          const u32x2 w = {pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
          *reinterpret_cast<u32x2*>(orow + dt * 16) = w;
        }
      }
    }
  };

  // ---- one key block against the current segment ---------------------------
  auto compute_block = [&](int buf, int kb) __attribute__((always_inline)) {
    const int key0 = kb * BN;
    const int wave_qmin = start_pos + seg_qb * C::BM + wave * RPW;
    if (key0 > wave_qmin + RPW - 1) return;   // every key of the block is in this wave's future
    const unsigned char* tk = tileK(buf);
    const unsigned char* tv = tileV(buf);
    // S^T = K Q^T; the K operands of k-step ks+1 are read while the MFMAs of
    // step ks run.
    auto load_k = [&](int ks, bf16x8_t* ka) __attribute__((always_inline)) {
#pragma unroll
      for (int kt = 0; kt < C::KT; ++kt) {
        const int r = kt * 16 + m16;
        ka[kt] = as_bf16x8(*reinterpret_cast<const u32x4*>(tk + r * C::RB + (((ks * 4 + g4) ^ swz<D>(r)) << 4)));
      }
    };
    f32x4 st[C::KT][C::QT];
#pragma unroll
    for (int kt = 0; kt < C::KT; ++kt)
#pragma unroll
      for (int qt = 0; qt < C::QT; ++qt) st[kt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    bf16x8_t ka0[C::KT], ka1[C::KT];
    load_k(0, ka0);
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      bf16x8_t* cur = (ks & 1) ? ka1 : ka0;
      bf16x8_t* nxt = (ks & 1) ? ka0 : ka1;
      if (ks + 1 < C::KS) load_k(ks + 1, nxt);
#pragma unroll
      for (int kt = 0; kt < C::KT; ++kt)
#pragma unroll
        for (int qt = 0; qt < C::QT; ++qt) st[kt][qt] = mfma16x16x32(cur[kt], qb_op[qt][ks], st[kt][qt]);
    }
    // V^T operands come from transposing LDS reads.
    const int vr = 4 * g4 + (m16 >> 2);          // row within a 32-key step (first half)
    const int vc = 4 * (m16 & 3);                // column offset within a 16-wide d tile
    auto load_v = [&](int s2, bf16x8_t* va) __attribute__((always_inline)) {
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) {
        const int d = dt * 16 + vc;
        const int r0 = s2 * 32 + vr, r1 = r0 + 16;
        const unsigned char* p0 = tv + r0 * C::RB + (((d >> 3) ^ swz<D>(r0)) << 4) + ((d & 7) << 1);
        const unsigned char* p1 = tv + r1 * C::RB + (((d >> 3) ^ swz<D>(r1)) << 4) + ((d & 7) << 1);
        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)p0);
        const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)p1);
        const u32x4 w = {__builtin_bit_cast(u32x2, lo)[0], __builtin_bit_cast(u32x2, lo)[1],
                         __builtin_bit_cast(u32x2, hi)[0], __builtin_bit_cast(u32x2, hi)[1]};
        va[dt] = as_bf16x8(w);
      }
    };
    // Mask (raw scores), row maxima and P^T operands. The masked variant is
    // only instantiated for blocks that reach the diagonal (a wave-uniform
    // branch; a select per element would cost every block).
    float alpha[C::QT];
    bool any_rescale = false;
    bf16x8_t pb[C::PS][C::QT];   // step s2 covers keys 32*s2 + {4g..4g+3, 16+4g..16+4g+3}
    float l_psum[C::QT];
    auto softmax = [&](const bool masked) __attribute__((always_inline)) {
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
#pragma unroll
      for (int qt = 0; qt < C::QT; ++qt) {
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < C::KT; ++kt)
#pragma unroll
          for (int j = 0; j < 4; ++j) mx = fmaxf(mx, st[kt][qt][j]);
        mx = xrow4_max(mx) * scale_log2;
        // Lazy rescaling: the reference max only moves when the block max
        // exceeds it by more than 2^8 (p <= 256 stays exact in fp32 and bf16
        // range); the normalisation by l is unaffected.
        const bool grow = mx > m_run[qt] + kLazyRescaleLog2;
        const float mn = grow ? mx : m_run[qt];
        alpha[qt] = grow ? ((m_run[qt] == -INFINITY) ? 0.f : fast_exp2(m_run[qt] - mn)) : 1.0f;
        m_run[qt] = mn;
        any_rescale |= grow;
      }
#pragma unroll
      for (int qt = 0; qt < C::QT; ++qt) {
        l_psum[qt] = 0.f;
        const float nm = -m_run[qt];
#pragma unroll
        for (int s2 = 0; s2 < C::PS; ++s2) {
          float p[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            p[j] = fast_exp2(fmaf(st[2 * s2][qt][j], scale_log2, nm));
            p[4 + j] = fast_exp2(fmaf(st[2 * s2 + 1][qt][j], scale_log2, nm));
          }
#pragma unroll
          for (int j = 0; j < 8; ++j) l_psum[qt] += p[j];
          const u32x4 w = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]),
                           pack_bf16x2(p[4], p[5]), pack_bf16x2(p[6], p[7])};
          pb[s2][qt] = as_bf16x8(w);
        }
      }
    };
    if (key0 + BN - 1 > wave_qmin) softmax(true);
    else softmax(false);
    if (__any(any_rescale)) {
#pragma unroll
      for (int qt = 0; qt < C::QT; ++qt) {
        l_run[qt] *= alpha[qt];
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) o_acc[dt][qt] *= alpha[qt];
      }
    }
#pragma unroll
    for (int qt = 0; qt < C::QT; ++qt) l_run[qt] += l_psum[qt];
    // O^T += V^T P^T, one 32-key step at a time.
#pragma unroll
    for (int s2 = 0; s2 < C::PS; ++s2) {
      bf16x8_t va[C::DT];
      load_v(s2, va);
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int qt = 0; qt < C::QT; ++qt) o_acc[dt][qt] = mfma16x16x32(va[dt], pb[s2][qt], o_acc[dt][qt]);
    }
  };

  // ---- main loop: both groups in lock step -----------------------------------
  if (my_n > 0) {
    begin_segment(qb_of(0));
    issue(0, kb_of(0));
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcntZero);
  __syncthreads();
  auto iteration = [&](int cur, int nxt, int it) __attribute__((always_inline)) {
    if (it + 1 < my_n) issue(nxt, kb_of(it + 1));
    if (it < my_n) {
      if (cache_head) write_cache(cur, kb_of(it), qb_of(it));
      compute_block(cur, kb_of(it));
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcntZero);   // the DMA into the other buffer has landed
    __syncthreads();
  };
  auto run = [&](int it0, int it1) __attribute__((always_inline)) {
    for (int it = it0; it < it1; ++it) iteration(it & 1, (it + 1) & 1, it);
  };
  // Two loops split at the light/heavy switch of group A, so no loop body
  // holds a Q reload.
  const int it_switch = (nl > 0 && hsplit > 0) ? nl : tA;
  run(0, it_switch);
  if (it_switch < tA) {
    if (grp == 0) {
      store_segment();
      begin_segment(qh);
    }
    run(it_switch, tA);
  }

  // ---- finish: light block of A, heavy block (merged when split) -------------
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

template <int D, int RPW, int BN>
int launch_prefill(const bf16* q, const bf16* k, const bf16* v, int kv_row_stride,
                   long kv_head_stride, bf16* out, int S, int start_pos, int Hq,
                   int Hkv, bf16* k_cache, bf16* v_cache, int cache_pos, int max_seq,
                   hipStream_t st) {
  using C = PrefillCfg<D, RPW, BN>;
  const int nqb = (S + C::BM - 1) / C::BM;
  const int npair = (nqb + 1) / 2;
  const float scale_log2 = kLog2e / sqrtf(static_cast<float>(D));
  hipLaunchKernelGGL((gqa_prefill_kernel<D, RPW, BN>), dim3(npair, Hq), dim3(2 * kThreads), 0, st,
                     q, Hq * D, k, v, kv_row_stride, kv_head_stride, out, Hq * D, S, start_pos,
                     Hkv, Hq / Hkv, scale_log2, k_cache, v_cache, cache_pos, max_seq);
  return check_launch("gqa_prefill");
}

int dispatch_prefill(int D, const bf16* q, const bf16* k, const bf16* v, int kv_row_stride,
                     long kv_head_stride, bf16* out, int S, int start_pos, int Hq, int Hkv,
                     bf16* k_cache, bf16* v_cache, int cache_pos, int max_seq, hipStream_t st) {
  switch (D) {
    case 64:
      return launch_prefill<64, 32, 64>(q, k, v, kv_row_stride, kv_head_stride, out, S, start_pos,
                                        Hq, Hkv, k_cache, v_cache, cache_pos, max_seq, st);
    case 128:
      return launch_prefill<128, 32, 64>(q, k, v, kv_row_stride, kv_head_stride, out, S, start_pos,
                                         Hq, Hkv, k_cache, v_cache, cache_pos, max_seq, st);
    case 256:
      return launch_prefill<256, 16, 32>(q, k, v, kv_row_stride, kv_head_stride, out, S, start_pos,
                                         Hq, Hkv, k_cache, v_cache, cache_pos, max_seq, st);
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

extern "C" int aila_hip_gqa_prefill_cached(const void* q, const void* k_cache, const void* v_cache,
                                           void* out, int S, int start_pos, int Hq, int Hkv, int D,
                                           int max_seq, void* stream) {
  using namespace aila;
  AILA_REQUIRE(q && k_cache && v_cache && out, "gqa_prefill_cached: null pointer");
  AILA_REQUIRE(S > 0 && start_pos >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq <= 65535,
               "gqa_prefill_cached: bad shape (S=%d start_pos=%d Hq=%d Hkv=%d)", S, start_pos, Hq, Hkv);
  AILA_REQUIRE(static_cast<long>(start_pos) + S <= max_seq,
               "gqa_prefill_cached: start_pos + S = %ld > max_seq=%d", static_cast<long>(start_pos) + S, max_seq);
  return dispatch_prefill(D, static_cast<const bf16*>(q), static_cast<const bf16*>(k_cache),
                          static_cast<const bf16*>(v_cache), D, static_cast<long>(max_seq) * D,
                          static_cast<bf16*>(out), S, start_pos, Hq, Hkv, nullptr, nullptr, 0, max_seq,
                          static_cast<hipStream_t>(stream));
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

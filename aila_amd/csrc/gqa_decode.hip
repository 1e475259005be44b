// Split-K flash-decode for single-token GQA over a bf16 KV cache (gfx950).
//
// Reference: ops::attention_decode (src/ops/AttentionOps.cpp:499-643) with
// its baseline kernel (:73-166) and the exact split/merge kernel for D=256
// (:168-320). One design serves every (D, group) here:
//
//  * Grid (split, kv_head, sequence). A workgroup (4 waves) owns a range of
//    `split_len` cache rows of one KV head and ALL G = Hq/Hkv query heads of
//    that group, so each K/V byte is read from HBM once per step.
//  * Scores on MFMA: v_mfma_f32_16x16x32_bf16 with A = the G query heads
//    (rows, zero padded to 16) and B = 16 cache rows. Lane l loads 16 bytes of
//    row (t0 + l%16) at byte offset 64*ks + 16*(l/16): each load instruction
//    reads 16 rows x 64 contiguous bytes, and lanes 0..15 receive the scores
//    of heads 0..3 for 16 tokens.
//  * Online softmax in the log2 domain; per-head block maxima are reduced
//    with DPP row operations inside the 16-lane row that holds the head.
//  * P.V on VALU: P goes through a small per-wave LDS slice; V rows are read
//    with coalesced 16-byte loads (D/8 lanes per row) and accumulated into
//    per-lane fp32 registers.
//  * Waves of a workgroup merge through LDS; a workgroup writes either the
//    final bf16 output (one split) or a partial record {m, l, acc[D]} in the
//    reference's layout (AttentionOps.cpp:50-51: [0]=m, [1]=l, [16..]=acc,
//    m in natural-log units), merged by gqa_decode_merge_kernel (:276-319).
#include "common.hpp"

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

namespace aila {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kChunk = 16;            // tokens per wave iteration (one MFMA column group)
constexpr int kNontemporal = 2;       // cache-policy bit for streamed K/V (read once)
// s_waitcnt immediate (gfx9 encoding): vmcnt = 0, expcnt and lgkmcnt not waited on.
constexpr int kWaitVmcntZero = 0x0F70;
constexpr int kMaxSplits = 256;
constexpr int kRecHeader = 16;

// Chunk swizzle of the per-wave K stage rows (16 rows x D/8 16-byte chunks):
// the 16 rows read by one MFMA operand load hit 16 distinct bank groups.
template <int D>
__device__ __forceinline__ int kswz(int r) {
  if constexpr (D >= 128) return r & 15;
  else return (r >> 1) & 7;
}

typedef __attribute__((address_space(3))) void lds_void_t;

// Fused decode preparation (decode_prepare_qkv[_partial] / qgkv_packed,
// ElementwiseOps.cpp:105-216, 555-863) applied inside the decode: q and the
// new k get per-head RMSNorm (rounded to bf16), then NeoX RoPE over the
// first `rot` dims at the token's position (rounded to bf16); the gate half
// of a packed q|gate head is copied to gate_out by split 0.
struct PrepArgs {
  int q_stride;          // elements between query heads of q_in (D, or 2D packed)
  const bf16* qn_w;      // [D] or null
  const bf16* kn_w;      // [D] or null
  bf16* gate_out;        // [B, Hq, D] (packed only) or null
  int apply_gate;        // packed only: out *= sigmoid(gate) instead of copying the gate out
  int rot;               // rotary dims, even, in [2, D]
  float eps;
  RopePos rope;          // rotary positions (zero: the cache row)
  RopeFreq freq;         // inverse frequencies of the rotary pairs
};

// Paged KV cache: the rows of sequence b live in fixed-size pages of a
// shared pool [num_pages, Hkv, page_size, D]; row t is row t % page_size of
// page table[b * max_pages + t / page_size]. page_size is a multiple of the
// 16-row chunk a wave loads, so a chunk never straddles two pages.
struct PageArgs {
  const int* table;      // [B, max_pages] device page indices
  int page_size;
  int max_pages;
};

// Decode window with attention sinks (ops::attention_decode's
// AILA_ATTN_DECODE_WINDOW / _WINDOW_START / _SINK knobs,
// AttentionOps.cpp:533-551, 598-616): once a sequence holds more than
// `start` rows it attends its first `sink` rows and its last `window` rows
// only. window = 0: off.
struct WinArgs {
  int window, start, sink;
};
// The attended rows of a sequence of L cached rows as a logical range
// [0, len): logical row t is cache row t below `sink` and t + gap above.
struct WinPlan {
  int len, sink, gap;
};
__host__ __device__ __forceinline__ WinPlan window_plan(int L, const WinArgs& w) {
  const bool apply = w.window > 0 && L > w.start;
  const int eff_window = apply ? (L < w.window ? L : w.window) : L;
  int tail = L - eff_window;
  int sink = 0;
  if (apply && w.sink > 0) sink = w.sink < tail ? w.sink : tail;
  int len = eff_window + sink;
  if (len >= L) {   // sink and tail meet: the whole context (AttentionOps.cpp:612-616)
    tail = 0;
    sink = 0;
    len = L;
  }
  return WinPlan{len, sink, tail - sink};
}

// Rows per split of one sequence. With a host length the host plan's
// split_len holds. With device lengths the launch is sized for a bound (the
// capacity a captured graph replays with), so the launched nsplit splits
// share the sequence's actual rows evenly instead, in whole 16-row chunks:
// no split then streams more than ~1/nsplit of the rows. The merge derives
// the same value.
__device__ __forceinline__ int split_rows(int len, int split_len, int nsplit, bool device_len) {
  if (!device_len) return split_len;
  const int per = (len + nsplit - 1) / nsplit;
  return max(kChunk, (per + kChunk - 1) / kChunk * kChunk);
}

template <int D, int G, bool PREP = false, bool PAGED = false, bool WIN = false>
__global__ __launch_bounds__(kThreads) void gqa_decode_split_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ kc,
    const bf16* __restrict__ vc, bf16* __restrict__ out,
    float* __restrict__ part, int Hq, int Hkv, int max_seq, int L,
    const int* __restrict__ seq_lens, int len_bias, int split_len, int nsplit_max, int group,
    float scale_log2, const bf16* __restrict__ k_new, const bf16* __restrict__ v_new, PrepArgs pa, PageArgs pg,
    WinArgs wn) {
  static_assert(D % 32 == 0 && D <= 256, "D");
  static_assert(!(PAGED && PREP), "the paged variant has no fused preparation");
  static_assert(!(WIN && (PAGED || PREP)), "the window variant is contiguous and has no fused append");
  static_assert(G == 1 || G == 2 || G == 4 || G == 8, "G");
  constexpr int KS = D / 32;          // MFMA k-steps over the head dim
  constexpr int VL = D / 8;           // lanes per V row (16 B each)
  constexpr int VR = 64 / VL;         // V rows per load instruction
  constexpr int GR = (G + 3) / 4;     // 16-lane rows holding score heads
  constexpr int NC = D / 8;           // 16-byte chunks per row
  constexpr int STAGE = kChunk * D * 2;          // bytes of one K stage (16 rows)
  constexpr int NDMA = STAGE / 1024;             // DMA instructions per stage per wave

  // Group of `group` = Hq/Hkv query heads per KV head, served G (the tile)
  // at a time: grid.y = Hkv * chunks, and the workgroup of chunk c of KV
  // head kvh holds query heads group*kvh + G*c .. + gv - 1 (gv <= G; rows of
  // the tile past gv are zero and their results unused).
  const int chunks = (group + G - 1) / G;
  const int split = blockIdx.x, b = blockIdx.z;
  const int kvh = static_cast<int>(blockIdx.y) / chunks;
  const int chunk = static_cast<int>(blockIdx.y) - kvh * chunks;
  const int gv = min(G, group - chunk * G);
  int len = L;
  if (seq_lens) len = min(max(seq_lens[b] + len_bias, 0), L);
  // window: logical row t reads cache row t (t < wsink) or t + wgap
  int wsink = 0, wgap = 0;
  if constexpr (WIN) {
    const WinPlan wp = window_plan(len, wn);
    len = wp.len;
    wsink = wp.sink;
    wgap = wp.gap;
  } else {
    (void)wn;
  }
  const int sl = split_rows(len, split_len, static_cast<int>(gridDim.x), seq_lens != nullptr);
  const int s0 = split * sl;
  const int nsplit_b = (len + sl - 1) / sl;
  const bool single = (part == nullptr);
  if (!single && split >= nsplit_b) return;   // the merge reads nsplit_b records
  const int s1 = min(s0 + sl, len);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m16 = lane & 15, g4 = lane >> 4;
  const size_t kv_off = PAGED ? 0 : (static_cast<size_t>(b) * Hkv + kvh) * max_seq * D;
  const bf16* K = kc + kv_off;
  const bf16* V = vc + kv_off;
  const int h0 = kvh * group + chunk * G;   // first query head of this workgroup
  // Element offset (from K / V) of cache row t0, the first row of a 16-row
  // chunk; rows t0 .. t0 + 15 follow it contiguously in both layouts.
  // `page` is the page holding t0 (paged layout only).
  auto row_off = [&](int t0, int page) __attribute__((always_inline)) -> size_t {
    if constexpr (PAGED) {
      const int in_page = t0 - (t0 / pg.page_size) * pg.page_size;
      const int pgu = __builtin_amdgcn_readfirstlane(page);
      return ((static_cast<size_t>(pgu) * Hkv + kvh) * pg.page_size + in_page) * D;
    } else {
      (void)page;
      return static_cast<size_t>(t0) * D;
    }
  };
  // page index of the chunk at t0 (uniform per wave). Branch-free: the
  // table index is clamped to the sequence's row of the table, so a lookup
  // for a chunk past the split reads a valid entry that is never used (an
  // early return for such chunks, a branch on a wave-uniform value the
  // compiler treats as divergent, measured wrong pages on gfx950).
  // The lookup is a vector buffer load, not a scalar load: scalar loads
  // share their wait counter with the LDS reads of the K operands, so a
  // pending page lookup would stall every LDS wait of the iteration (measured
  // 7% slower); the vector load completes under the iteration's own vmcnt wait.
  const __amdgpu_buffer_rsrc_t tab_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int*>(PAGED ? pg.table + static_cast<size_t>(b) * pg.max_pages : nullptr), 0,
      PAGED ? pg.max_pages * 4 : 0, kBufferRsrcWord3);
  auto page_of = [&](int t0) __attribute__((always_inline)) -> int {
    if constexpr (PAGED) {
      const int pi = min(t0 / pg.page_size, pg.max_pages - 1);
      return __builtin_amdgcn_raw_buffer_load_b32(tab_rsrc, pi * 4, 0, 0);
    } else {
      (void)t0;
      return 0;
    }
  };

  __shared__ __attribute__((aligned(1024))) unsigned char s_k[kWaves][2][STAGE];
  __shared__ float s_p[kWaves][kChunk][G];
  __shared__ float s_ml[kWaves][2][G];
  __shared__ float s_q[PREP ? G : 1][PREP ? D : 1];   // prepared q (fused preparation only)
  __shared__ float s_tab[PREP ? D : 1];               // (cos, sin) per rotary pair
  static_assert(sizeof(float) * kWaves * G * D <= sizeof(s_k), "epilogue reuses the K ring");
  // epilogue: per-wave accumulators, in the (then idle) K ring
  float (*s_acc)[G][D] = reinterpret_cast<float (*)[G][D]>(&s_k[0][0][0]);

  // K rows of one 16-token chunk -> this wave's LDS stage, whole rows per
  // DMA instruction (lane order within a row follows the swizzle).
  auto dma_k = [&](int stage, int t0, int page) __attribute__((always_inline)) {
    unsigned char* dst = s_k[wave][stage];
    const bf16* Kc = K + row_off(t0, page);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int p = i * 64 + lane;
      const int r = p / NC, qc = (p % NC) ^ kswz<D>(r);
      const int tok = min(t0 + r, s1 - 1) - t0;
      const bf16* src;
      if constexpr (WIN) {
        const int t = t0 + tok;
        src = K + static_cast<size_t>(t < wsink ? t : t + wgap) * D + qc * 8;
      } else {
        src = Kc + static_cast<size_t>(tok) * D + qc * 8;
      }
      __builtin_amdgcn_global_load_lds(src, (lds_void_t*)(dst + i * 1024), 16, 0, kNontemporal);
    }
  };

  // The first chunk's K DMA goes out before the query work whenever that
  // chunk cannot hold the row this launch appends (fused preparation).
  int t0 = s0 + wave * kChunk;
  int pg_cur = page_of(t0);
  const bool early = PREP && t0 < s1 && t0 + kChunk <= len - 1;
  if (early) dma_k(0, t0, pg_cur);

  // Query operand (A rows = heads, zero rows for m16 >= G).
  bf16x8_t qa[KS];
  if constexpr (!PREP) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (m16 < gv) raw = ld16(q + (static_cast<size_t>(b) * Hq + h0 + m16) * D + ks * 32 + g4 * 8);
      qa[ks] = as_bf16x8(raw);
    }
  } else {
    // Prepared q, computed once per workgroup: wave w normalises heads w and
    // w + 4 (one wave per head, D/64 dims per lane), the RoPE pass rotates
    // pairs in place, and every wave then reads its A operands from LDS.
    const int half = pa.rot / 2;
    const RowPos rp = rope_row_pos(pa.rope, b, len - 1);
    for (int j = threadIdx.x; j < half; j += kThreads) {
      const float freq = rope_inv_freq(pa.rope, pa.freq, j);
      const float ang = rope_freq_pos(rp, j) * freq;
      s_tab[2 * j] = cosf(ang);
      s_tab[2 * j + 1] = sinf(ang);
    }
    constexpr int E = D / 64;
#pragma unroll
    for (int hh = wave; hh < gv; hh += kWaves) {
      const bf16* qr = q + (static_cast<size_t>(b) * Hq + h0 + hh) * pa.q_stride;
      float xv[E], ss = 0.f;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        xv[i] = bf2f(qr[lane + 64 * i]);
        ss = fmaf(xv[i], xv[i], ss);
      }
      ss = wave_sum(ss);
      const float rms = sqrtf(ss / static_cast<float>(D) + pa.eps);
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const int d = lane + 64 * i;
        const float w = pa.qn_w ? bf2f(pa.qn_w[d]) : 1.0f;
        s_q[hh][d] = bf2f(f2bf((xv[i] / rms) * w));
      }
      // packed q|gate: split 0 copies the gate half through
      if (pa.gate_out != nullptr && split == 0)
        for (int d = lane; d < D; d += 64)
          pa.gate_out[(static_cast<size_t>(b) * Hq + h0 + hh) * D + d] = qr[D + d];
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < gv * half; idx += kThreads) {
      const int hh = idx / half, j = idx % half;
      const float x0 = s_q[hh][j], x1 = s_q[hh][j + half];
      const float c = s_tab[2 * j], sn = s_tab[2 * j + 1];
      s_q[hh][j] = bf2f(f2bf(x0 * c - x1 * sn));
      s_q[hh][j + half] = bf2f(f2bf(x1 * c + x0 * sn));
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (m16 < gv) {
        const float* r = &s_q[m16][ks * 32 + g4 * 8];
        w = u32x4{pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]), pack_bf16x2(r[4], r[5]),
                  pack_bf16x2(r[6], r[7])};
      }
      qa[ks] = as_bf16x8(w);
    }
  }

  float m_run[G], l_part[G], acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m_run[h] = -INFINITY;
    l_part[h] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  }
  const int vd = (lane % VL) * 8;
  const int vr = lane / VL;

  // Fused append (decode_prepare's cache write): the workgroup owning the
  // last row writes the new token's K and V there before anything reads it.
  if (PREP && len > 0 && split == nsplit_b - 1) {
    // the new k row: RMSNorm + RoPE at row len-1, staged through wave 0's
    // second K stage (untouched until the loop), then k and v rows written
    if (wave == 0) {
      float* sx = reinterpret_cast<float*>(&s_k[0][1][0]);
      static_assert(STAGE >= D * sizeof(float), "k staging fits");
      const bf16* kr = k_new + (static_cast<size_t>(b) * Hkv + kvh) * D;
      constexpr int E = D / 64;
      float xv[E], ss = 0.f;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        xv[i] = bf2f(kr[lane + 64 * i]);
        ss = fmaf(xv[i], xv[i], ss);
      }
      ss = wave_sum(ss);
      const float rms = sqrtf(ss / static_cast<float>(D) + pa.eps);
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const int d = lane + 64 * i;
        const float w = pa.kn_w ? bf2f(pa.kn_w[d]) : 1.0f;
        sx[d] = bf2f(f2bf((xv[i] / rms) * w));
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int p = len - 1, half = pa.rot / 2;
      const float* tab = s_tab;
      bf16* krow = const_cast<bf16*>(K) + static_cast<size_t>(p) * D;
      bf16* vrow = const_cast<bf16*>(V) + static_cast<size_t>(p) * D;
      const bf16* vsrc = v_new + (static_cast<size_t>(b) * Hkv + kvh) * D;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const int d = lane + 64 * i;
        float r = sx[d];
        if (d < pa.rot) {
          const int dd = d < half ? d : d - half;
          const float c = tab[2 * dd], sn = tab[2 * dd + 1];
          r = d < half ? sx[d] * c - sx[d + half] * sn : sx[d] * c + sx[d - half] * sn;
        }
        krow[d] = f2bf(r);
        vrow[d] = vsrc[d];
      }
      __builtin_amdgcn_s_waitcnt(kWaitVmcntZero);
    }
    __syncthreads();
  } else if (!PAGED && k_new != nullptr && len > 0 && split == nsplit_b - 1) {
    if (wave == 0 && lane < 2 * NC) {
      const int row = len - 1;
      const bool isv = lane >= NC;
      const int c = isv ? lane - NC : lane;
      const bf16* src = (isv ? v_new : k_new) + (static_cast<size_t>(b) * Hkv + kvh) * D + c * 8;
      bf16* dst = const_cast<bf16*>(isv ? V : K) + static_cast<size_t>(row) * D + c * 8;
      *reinterpret_cast<u32x4*>(dst) = ld16(src);
      __builtin_amdgcn_s_waitcnt(kWaitVmcntZero);
    }
    __syncthreads();
  }

  if (!early && t0 < s1) dma_k(0, t0, pg_cur);
  // The loop reads a chunk's K stage at its top; every iteration waits for
  // its own DMA at its end, and this wait covers the first chunk. The
  // compiler does not order that first LDS read after the DMA by itself: the
  // rotated loop of the fused-preparation kernel read the stage before it
  // landed (stale LDS from the previous workgroup).
  __builtin_amdgcn_s_waitcnt(kWaitVmcntZero);
  int pg_nxt = page_of(t0 + kWaves * kChunk);
  for (int it = 0; t0 < s1; ++it, t0 += kWaves * kChunk) {
    const int stage = it & 1;
    // ---- K operands of this chunk (its DMA was issued one chunk earlier) --
    const unsigned char* ks_base = s_k[wave][stage];
    u32x4 kb[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      kb[ks] = *reinterpret_cast<const u32x4*>(ks_base + m16 * (D * 2) + (((ks * 4 + g4) ^ kswz<D>(m16)) << 4));
    // ---- V rows of this chunk: nontemporal register loads, issued before
    //      the next K DMA so waiting on V never waits on that prefetch ------
    u32x4 vv[kChunk / VR];
    const bf16* Vc = V + row_off(t0, pg_cur);
#pragma unroll
    for (int i = 0; i < kChunk / VR; ++i) {
      const int tok = min(t0 + vr + i * VR, s1 - 1) - t0;
      const bf16* src;
      if constexpr (WIN) {
        const int t = t0 + tok;
        src = V + static_cast<size_t>(t < wsink ? t : t + wgap) * D + vd;
      } else {
        src = Vc + static_cast<size_t>(tok) * D + vd;
      }
      vv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
    }
    const int t_next = t0 + kWaves * kChunk;
    if (t_next < s1) dma_k(stage ^ 1, t_next, pg_nxt);
    // the page of the chunk after next goes out now, used one iteration later
    const int pg_nn = page_of(t_next + kWaves * kChunk);
    pg_cur = pg_nxt;
    pg_nxt = pg_nn;
    // ---- scores on MFMA ------------------------------------------------------
    f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) c = mfma16x16x32(qa[ks], as_bf16x8(kb[ks]), c);
    const bool valid = (t0 + m16) < s1;
    float sc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) sc[j] = valid ? c[j] * scale_log2 : -INFINITY;
    // ---- online softmax (log2 domain) ---------------------------------------
    float alpha[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const int j = h & 3, row = h >> 2;
      float bm = row16_max(sc[j]);
      bm = readlane_f(bm, row * 16);
      const float mn = fmaxf(m_run[h], bm);
      alpha[h] = (m_run[h] == -INFINITY) ? 0.f : fast_exp2(m_run[h] - mn);
      m_run[h] = mn;
      l_part[h] *= alpha[h];
    }
    // p for the heads held by this lane's row; write to the wave's P slice.
#pragma unroll
    for (int r = 0; r < GR; ++r) {
      if (g4 == r) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int h = r * 4 + j;
          if (h < G) {
            const float mref = (m_run[h] == -INFINITY) ? 0.f : m_run[h];
            const float p = fast_exp2(sc[j] - mref);
            l_part[h] += p;
            s_p[wave][m16][h] = p;
          }
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- P.V ------------------------------------------------------------------
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] *= alpha[h];
    }
#pragma unroll
    for (int i = 0; i < kChunk / VR; ++i) {
      float vf[8];
      unpack8(vv[i], vf);
      float p[G];
#pragma unroll
      for (int h = 0; h < G; ++h) p[h] = s_p[wave][vr + i * VR][h];
#pragma unroll
      for (int h = 0; h < G; ++h) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] += p[h] * vf[e];
      }
    }
    // The next iteration overwrites this wave's P slice and reads the other
    // K stage, whose DMA must have landed.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    __builtin_amdgcn_s_waitcnt(kWaitVmcntZero);
  }

  // ---- wave epilogue --------------------------------------------------
  // l: per-lane partial sums live in the 16-lane row that owns the head.
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const int row = h >> 2;
    float l = row16_sum(l_part[h]);
    l = readlane_f(l, row * 16);
    l_part[h] = l;
  }
  // Sum acc over the VR row phases (lanes with equal vd).
#pragma unroll
  for (int h = 0; h < G; ++h) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = acc[h][e];
#pragma unroll
      for (int off = VL; off < 64; off <<= 1) x += __shfl_xor(x, off);
      acc[h][e] = x;
    }
  }
  __syncthreads();   // every wave is done with the K ring before it becomes s_acc
  if (vr == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s_acc[wave][h][vd + e] = acc[h][e];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      s_ml[wave][0][h] = m_run[h];
      s_ml[wave][1][h] = l_part[h];
    }
  }
  __syncthreads();

  // ---- workgroup merge ------------------------------------------------
  for (int idx = threadIdx.x; idx < gv * D; idx += kThreads) {
    const int h = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_ml[w][0][h]);
    float A = 0.f, Ls = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = s_ml[w][0][h];
      const float f = (mw == -INFINITY) ? 0.f : fast_exp2(mw - M);
      A += f * s_acc[w][h][d];
      Ls += f * s_ml[w][1][h];
    }
    const int hq = h0 + h;
    if (single) {
      float o = Ls > 0.f ? A / Ls : 0.f;
      if (PREP && pa.apply_gate) {   // gated attention: out * sigmoid(gate) (ElementwiseOps.cpp:519-553)
        const float g = bf2f(q[(static_cast<size_t>(b) * Hq + hq) * pa.q_stride + D + d]);
        o *= 1.0f / (1.0f + expf(-g));
      }
      out[(static_cast<size_t>(b) * Hq + hq) * D + d] = f2bf(o);
    } else {
      float* rec = part + ((static_cast<size_t>(b) * Hq + hq) * nsplit_max + split) * (kRecHeader + D);
      rec[kRecHeader + d] = A;
      if (d == 0) {
        rec[0] = (M == -INFINITY) ? -INFINITY : M * (1.0f / kLog2e);
        rec[1] = Ls;
      }
    }
  }
}

// Merge of split records, AttentionOps.cpp:276-319: M = max m_i,
// out = sum_i e^(m_i - M) acc_i / sum_i e^(m_i - M) l_i.
// Thread t owns 4 head dims (float4 column c) of the splits i = part (mod P),
// so its record reads are independent and issued together; the P partial
// sums meet in LDS.
template <int D, bool WIN = false>
__global__ __launch_bounds__(256) void gqa_decode_merge_kernel(
    const float* __restrict__ part, bf16* __restrict__ out, int Hq, int L,
    const int* __restrict__ seq_lens, int len_bias, int split_len, int nsplit, int nsplit_max,
    const bf16* __restrict__ gate, int gate_stride, WinArgs wn) {
  constexpr int C4 = D / 4;             // float4 columns
  constexpr int P = 256 / C4;           // split phases
  const int hq = blockIdx.x, b = blockIdx.y;
  int len = L;
  if (seq_lens) len = min(max(seq_lens[b] + len_bias, 0), L);
  if constexpr (WIN) len = window_plan(len, wn).len;
  else (void)wn;
  const int sl = split_rows(len, split_len, nsplit, seq_lens != nullptr);
  const int ns = (len + sl - 1) / sl;
  const float* rec0 = part + (static_cast<size_t>(b) * Hq + hq) * nsplit_max * (kRecHeader + D);
  __shared__ float s_f[kMaxSplits];
  __shared__ float s_inv;
  __shared__ f32x4 s_red[P][C4];
  const int c = threadIdx.x % C4, ph = threadIdx.x / C4;
  constexpr int U = 8;
  // This thread's accumulator rows of the first P*U splits go out before the
  // split factors, so the two rounds of loads overlap.
  auto load_acc = [&](int i0, f32x4 (&v)[U]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * P;
      v[u] = (i < ns) ? *reinterpret_cast<const f32x4*>(rec0 + static_cast<size_t>(i) * (kRecHeader + D) + kRecHeader + 4 * c)
                      : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  f32x4 v[U];
  load_acc(ph, v);
  // One wave computes the split factors (m and l of each record in one
  // load round: at most kMaxSplits / 64 records per lane).
  if (threadIdx.x < 64) {
    constexpr int kPerLane = kMaxSplits / 64;
    float mv[kPerLane], lv[kPerLane];
    float M = -INFINITY;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      const int i = threadIdx.x + 64 * j;
      mv[j] = -INFINITY;
      lv[j] = 0.f;
      if (i < ns) {
        const float* r = rec0 + static_cast<size_t>(i) * (kRecHeader + D);
        mv[j] = r[0];
        lv[j] = r[1];
      }
      M = fmaxf(M, mv[j]);
    }
    M = fmaxf(M, __shfl_xor(M, 32));
    M = fmaxf(M, __shfl_xor(M, 16));
    M = row16_max(M);
    float Ls = 0.f;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      const int i = threadIdx.x + 64 * j;
      const float f = (mv[j] == -INFINITY) ? 0.f : expf(mv[j] - M);
      if (i < ns) s_f[i] = f;
      Ls += f * lv[j];
    }
    Ls = wave_sum(Ls);
    if (threadIdx.x == 0) s_inv = Ls > 0.f ? 1.0f / Ls : 0.f;
  }
  __syncthreads();
  f32x4 a = {0.f, 0.f, 0.f, 0.f};
  for (int i0 = ph;; ) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * P;
      if (i < ns) a += s_f[i] * v[u];
    }
    i0 += P * U;
    if (i0 >= ns) break;
    load_acc(i0, v);
  }
  s_red[ph][c] = a;
  __syncthreads();
  if (threadIdx.x < C4) {
    f32x4 r = s_red[0][threadIdx.x];
#pragma unroll
    for (int p2 = 1; p2 < P; ++p2) r += s_red[p2][threadIdx.x];
    r *= s_inv;
    if (gate != nullptr) {   // gated attention: out * sigmoid(gate) (ElementwiseOps.cpp:519-553)
      const bf16* gr = gate + (static_cast<size_t>(b) * Hq + hq) * gate_stride + 4 * threadIdx.x;
#pragma unroll
      for (int j = 0; j < 4; ++j) r[j] *= 1.0f / (1.0f + expf(-bf2f(gr[j])));
    }
    const u32x2 w = {pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3])};
    *reinterpret_cast<u32x2*>(out + (static_cast<size_t>(b) * Hq + hq) * D + 4 * threadIdx.x) = w;
  }
}

// Launch arguments shared by the decode entry points.
struct DecodeArgs {
  const bf16* q;
  const bf16* kc;
  const bf16* vc;
  bf16* out;
  float* part;
  int B, Hq, Hkv, max_seq, L;
  const int* seq_lens;
  int len_bias;          // sequence b attends min(seq_lens[b] + len_bias, L) rows
  int split_len, nsplit, nsplit_max;
  int group, chunks;     // Hq / Hkv, and workgroups per KV head (group / tile, rounded up)
  const bf16* k_new;     // fused append (null: none)
  const bf16* v_new;
  PrepArgs prep;         // q_stride = 0: no fused preparation
  PageArgs pages;        // table = null: contiguous [B, Hkv, max_seq, D] cache
  WinArgs win;           // window = 0: every row
};

template <int D, int G>
int launch_decode(const DecodeArgs& a, hipStream_t st) {
  const float scale_log2 = kLog2e / sqrtf(static_cast<float>(D));
  const bool win = a.win.window > 0;
  if (a.prep.q_stride > 0)
    hipLaunchKernelGGL((gqa_decode_split_kernel<D, G, true>), dim3(a.nsplit, a.Hkv * a.chunks, a.B), dim3(kThreads), 0, st,
                       a.q, a.kc, a.vc, a.out, a.part, a.Hq, a.Hkv, a.max_seq, a.L, a.seq_lens, a.len_bias,
                       a.split_len, a.nsplit_max, a.group, scale_log2, a.k_new, a.v_new, a.prep, a.pages, a.win);
  else if (a.pages.table != nullptr)
    hipLaunchKernelGGL((gqa_decode_split_kernel<D, G, false, true>), dim3(a.nsplit, a.Hkv * a.chunks, a.B), dim3(kThreads), 0,
                       st, a.q, a.kc, a.vc, a.out, a.part, a.Hq, a.Hkv, a.max_seq, a.L, a.seq_lens, a.len_bias,
                       a.split_len, a.nsplit_max, a.group, scale_log2, a.k_new, a.v_new, a.prep, a.pages, a.win);
  else if (win)
    hipLaunchKernelGGL((gqa_decode_split_kernel<D, G, false, false, true>), dim3(a.nsplit, a.Hkv * a.chunks, a.B),
                       dim3(kThreads), 0, st, a.q, a.kc, a.vc, a.out, a.part, a.Hq, a.Hkv, a.max_seq, a.L,
                       a.seq_lens, a.len_bias, a.split_len, a.nsplit_max, a.group, scale_log2, a.k_new, a.v_new, a.prep,
                       a.pages, a.win);
  else
    hipLaunchKernelGGL((gqa_decode_split_kernel<D, G>), dim3(a.nsplit, a.Hkv * a.chunks, a.B), dim3(kThreads), 0, st,
                       a.q, a.kc, a.vc, a.out, a.part, a.Hq, a.Hkv, a.max_seq, a.L, a.seq_lens, a.len_bias,
                       a.split_len, a.nsplit_max, a.group, scale_log2, a.k_new, a.v_new, a.prep, a.pages, a.win);
  if (a.part) {
    const bool gated = a.prep.q_stride > 0 && a.prep.apply_gate;
    if (win)
      hipLaunchKernelGGL((gqa_decode_merge_kernel<D, true>), dim3(a.Hq, a.B), dim3(256), 0, st, a.part, a.out, a.Hq,
                         a.L, a.seq_lens, a.len_bias, a.split_len, a.nsplit, a.nsplit_max, nullptr, 0, a.win);
    else
      hipLaunchKernelGGL((gqa_decode_merge_kernel<D>), dim3(a.Hq, a.B), dim3(256), 0, st, a.part, a.out, a.Hq,
                         a.L, a.seq_lens, a.len_bias, a.split_len, a.nsplit, a.nsplit_max,
                         gated ? a.q + D : nullptr, a.prep.q_stride, a.win);
  }
  return check_launch("gqa_decode");
}

// Query-head tile of the split kernel for a group of g query heads per KV
// head: the smallest of 1, 2, 4, 8 that holds it, else 8 (several
// workgroups per KV head, each streaming its K/V; see the kernel).
int decode_tile(int g) { return g <= 1 ? 1 : g <= 2 ? 2 : g <= 4 ? 4 : 8; }

// Workgroups of the split kernel that the device holds at once (occupancy x
// CUs), per device, computed on first use. The split count targets exactly
// one such round: with L=32768, B=8, Hkv=4, D=256 measured 6.45 TB/s for
// 512 workgroups (2 per CU) against 5.91 for 2048 and 5.97 for 768 (every
// extra round pays the workgroup start-up latency and a partial tail).
// The per-device value is idempotent, so concurrent first calls may both
// compute it; the atomic makes the publication race-free.
template <int D, int G>
int resident_workgroups() {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cache[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 512;
  const int known = cache[dev].load(std::memory_order_relaxed);
  if (known > 0) return known;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gqa_decode_split_kernel<D, G>, kThreads, 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu <= 0 || cus <= 0)
    return 512;
  cache[dev].store(per_cu * cus, std::memory_order_relaxed);
  return per_cu * cus;
}

int resident_for(int D, int G) {
  auto pick = [&](auto d_tag) -> int {
    constexpr int DD = decltype(d_tag)::value;
    switch (decode_tile(G)) {
      case 1: return resident_workgroups<DD, 1>();
      case 2: return resident_workgroups<DD, 2>();
      case 4: return resident_workgroups<DD, 4>();
      case 8: return resident_workgroups<DD, 8>();
      default: return 512;
    }
  };
  switch (D) {
    case 64: return pick(std::integral_constant<int, 64>{});
    case 128: return pick(std::integral_constant<int, 128>{});
    case 256: return pick(std::integral_constant<int, 256>{});
    default: return 512;
  }
}

template <int D>
int dispatch_g(const DecodeArgs& a, hipStream_t st) {
  switch (decode_tile(a.group)) {
    case 1: return launch_decode<D, 1>(a, st);
    case 2: return launch_decode<D, 2>(a, st);
    case 4: return launch_decode<D, 4>(a, st);
    default: return launch_decode<D, 8>(a, st);
  }
}

// Validation, split planning and dispatch for both decode entry points.
int gqa_decode_impl(const void* q, const void* k_cache, const void* v_cache, void* out, void* workspace,
                    size_t workspace_bytes, int B, int Hq, int Hkv, int D, int max_seq, int cached_len,
                    const int* seq_lens, int len_bias, const void* k_new, const void* v_new,
                    hipStream_t st, const PrepArgs* prep = nullptr, const PageArgs* pages = nullptr,
                    const WinArgs* win = nullptr) {
  AILA_REQUIRE(q && k_cache && v_cache && out, "gqa_decode: null pointer");
  AILA_REQUIRE(B > 0 && B <= 65535 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 &&
                   static_cast<long>(Hkv) * ((Hq / Hkv + decode_tile(Hq / Hkv) - 1) / decode_tile(Hq / Hkv)) <= 65535,
               "gqa_decode: bad heads/batch (B=%d Hq=%d Hkv=%d)", B, Hq, Hkv);
  AILA_REQUIRE(cached_len >= 0 && cached_len <= max_seq,
               "gqa_decode: cached_len=%d outside [0, max_seq=%d]", cached_len, max_seq);
  DecodeArgs a{};
  a.q = static_cast<const bf16*>(q);
  a.kc = static_cast<const bf16*>(k_cache);
  a.vc = static_cast<const bf16*>(v_cache);
  a.out = static_cast<bf16*>(out);
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.max_seq = max_seq; a.L = cached_len;
  a.group = Hq / Hkv;
  a.chunks = (a.group + decode_tile(a.group) - 1) / decode_tile(a.group);
  a.seq_lens = seq_lens; a.len_bias = len_bias;
  a.k_new = static_cast<const bf16*>(k_new);
  a.v_new = static_cast<const bf16*>(v_new);
  a.prep = prep ? *prep : PrepArgs{};
  a.pages = pages ? *pages : PageArgs{};
  a.win = win ? *win : WinArgs{};
  // the split plan covers the rows a sequence of the bound length attends
  // (the window's attended count never decreases with the length)
  const int plan_len = a.win.window > 0 ? window_plan(cached_len, a.win).len : cached_len;
  // Records per (sequence, head) that the workspace holds; the split count
  // adapts to it (the reference's [Hq, max_tiles, 272] partials buffer for
  // D=256 is accepted as-is).
  const size_t rec_bytes = static_cast<size_t>(B) * Hq * (kRecHeader + D) * sizeof(float);
  a.nsplit_max = workspace ? static_cast<int>(std::min<size_t>(workspace_bytes / rec_bytes, kMaxSplits)) : 0;
  if (workspace && a.nsplit_max < 2)
    return set_error(AILA_HIP_EWORKSPACE, "gqa_decode: workspace %zu bytes holds < 2 split records (%zu bytes each)",
                     workspace_bytes, rec_bytes);
  // Short contexts run single-pass even with a workspace: up to two 16-row
  // chunks per wave (128 rows; 256 at D <= 128, where a chunk costs less)
  // one launch beats split + merge (graph replay, B=1 Hq=16 Hkv=8 D=128:
  // 4.2 against 6.5 us at 128 rows, 5.6 against 6.6 at 256; D=256 Hkv=4:
  // 7.1 against 8.3 at 128 rows, the split ahead from 192).
  const int single_max = D <= 128 ? 4 * kWaves * kChunk : 2 * kWaves * kChunk;
  if (plan_len == 0) {
    // Nothing to attend: the single-pass kernel writes a zero output.
    a.split_len = 1;
    a.nsplit = 1;
  } else if (workspace && plan_len <= single_max) {
    a.split_len = plan_len;
    a.nsplit = 1;
  } else if (workspace) {
    // One round of resident workgroups; splits are multiples of 64 rows
    // (one 16-row chunk per wave). Short contexts get one chunk per wave:
    // config 1 (512 rows, 8 KV heads) takes 6.4 us in 8 splits of 64 rows
    // against 7.1 us in 4 of 128.
    const int groups = B * Hkv * a.chunks;   // workgroups per split
    const int resident = resident_for(D, Hq / Hkv);
    int want = (resident + groups - 1) / groups;
    want = std::max(1, std::min(want, a.nsplit_max));
    a.split_len = (plan_len + want - 1) / want;
    a.split_len = ((a.split_len + kWaves * kChunk - 1) / (kWaves * kChunk)) * (kWaves * kChunk);
    // A context of 4096 rows or more that this leaves at one chunk per wave
    // (few sequences and KV heads) streams better in two-chunk splits: each
    // split's start-up then covers twice the rows (B=1, Hq=16, Hkv=4,
    // D=256, L=8192: 15.0 -> 12.8 us; Hq=32, Hkv=8, D=128, L=4096: 10.1 ->
    // 9.5 us). Shorter contexts keep one chunk per wave (config 1).
    if (a.split_len < 2 * kWaves * kChunk && plan_len >= 4096) a.split_len = 2 * kWaves * kChunk;
    a.nsplit = (plan_len + a.split_len - 1) / a.split_len;
    if (a.nsplit > 1) a.part = static_cast<float*>(workspace);   // one split: direct output
  } else {
    a.split_len = plan_len;
    a.nsplit = 1;
  }
  switch (D) {
    case 64: return dispatch_g<64>(a, st);
    case 128: return dispatch_g<128>(a, st);
    case 256: return dispatch_g<256>(a, st);
    default: return set_error(AILA_HIP_EUNSUPPORTED, "gqa_decode: D=%d not in {64,128,256}", D);
  }
}

}  // namespace
}  // namespace aila

extern "C" size_t aila_hip_gqa_decode_workspace_size(int B, int Hq, int D) {
  if (B <= 0 || Hq <= 0 || D <= 0) return 0;
  return static_cast<size_t>(B) * Hq * aila::kMaxSplits * (aila::kRecHeader + D) * sizeof(float);
}

extern "C" int aila_hip_gqa_decode(const void* q, const void* k_cache, const void* v_cache, void* out,
                                   void* workspace, size_t workspace_bytes, int B, int Hq, int Hkv, int D,
                                   int max_seq, int cached_len, const int* seq_lens, void* stream) {
  return aila::gqa_decode_impl(q, k_cache, v_cache, out, workspace, workspace_bytes, B, Hq, Hkv, D, max_seq,
                               cached_len, seq_lens, 0, nullptr, nullptr, static_cast<hipStream_t>(stream));
}

extern "C" int aila_hip_gqa_decode_window(const void* q, const void* k_cache, const void* v_cache, void* out,
                                          void* workspace, size_t workspace_bytes, int B, int Hq, int Hkv, int D,
                                          int max_seq, int cached_len, const int* seq_lens, int window,
                                          int window_start, int sink, void* stream) {
  using namespace aila;
  AILA_REQUIRE(window >= 0, "gqa_decode_window: window=%d < 0", window);
  WinArgs w{window, window_start < 0 ? std::max(512, window) : window_start, std::max(0, sink)};
  return gqa_decode_impl(q, k_cache, v_cache, out, workspace, workspace_bytes, B, Hq, Hkv, D, max_seq, cached_len,
                         seq_lens, 0, nullptr, nullptr, static_cast<hipStream_t>(stream), nullptr, nullptr, &w);
}

extern "C" int aila_hip_gqa_decode_paged(const void* q, const void* k_pages, const void* v_pages, void* out,
                                         void* workspace, size_t workspace_bytes, int B, int Hq, int Hkv, int D,
                                         int page_size, const int* block_table, int max_pages, int max_len,
                                         const int* seq_lens, void* stream) {
  using namespace aila;
  AILA_REQUIRE(block_table && seq_lens, "gqa_decode_paged: block_table and seq_lens are required");
  AILA_REQUIRE(page_size > 0 && page_size % kChunk == 0,
               "gqa_decode_paged: page_size=%d must be a positive multiple of %d", page_size, kChunk);
  AILA_REQUIRE(max_pages > 0 && static_cast<long>(max_pages) * page_size <= (1L << 30),
               "gqa_decode_paged: bad max_pages=%d", max_pages);
  const int max_seq = max_pages * page_size;
  AILA_REQUIRE(max_len >= 0 && max_len <= max_seq, "gqa_decode_paged: max_len=%d outside [0, %d]", max_len,
               max_seq);
  PageArgs pg{block_table, page_size, max_pages};
  return gqa_decode_impl(q, k_pages, v_pages, out, workspace, workspace_bytes, B, Hq, Hkv, D, max_seq, max_len,
                         seq_lens, 0, nullptr, nullptr, static_cast<hipStream_t>(stream), nullptr, &pg);
}

// ---------------------------------------------------------------------------
// Allocation-free decode: the split records live in a file-scope device
// array instead of a caller workspace. Its host-side name is only a stand-in
// for the symbol, so every host use goes through the device address that
// hipGetSymbolAddress returns, looked up once per device with that device
// current and kept per device.
namespace aila {
namespace {
constexpr size_t kScratchBytes = size_t(8) << 20;   // 8 MiB per device
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxScratchDev = 64;
std::atomic<float*> g_scratch_ptr[kMaxScratchDev];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (null + error set on
// failure).
float* scratch_for_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDev) {
    set_error(AILA_HIP_ELAUNCH, "gqa_decode_noalloc: no usable current device (%d)", dev);
    return nullptr;
  }
  float* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
  if (p) return p;
  void* addr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || addr == nullptr) {
    set_error(AILA_HIP_ELAUNCH, "gqa_decode_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
              hipGetErrorString(e));
    return nullptr;
  }
  p = static_cast<float*>(addr);
  g_scratch_ptr[dev].store(p, std::memory_order_release);
  return p;
}
}  // namespace
}  // namespace aila

extern "C" size_t aila_hip_gqa_decode_noalloc_max_bytes(void) { return aila::kScratchBytes; }

extern "C" int aila_hip_gqa_decode_noalloc(const void* q, const void* k_cache, const void* v_cache, void* out,
                                           int B, int Hq, int Hkv, int D, int max_seq, int cached_len,
                                           const int* seq_lens, void* stream) {
  using namespace aila;
  AILA_REQUIRE(B > 0 && Hq > 0 && D > 0, "gqa_decode_noalloc: bad shape (B=%d Hq=%d D=%d)", B, Hq, D);
  // Two split records per (sequence, head) is the least a split needs.
  const size_t need = static_cast<size_t>(B) * Hq * 2 * (kRecHeader + D) * sizeof(float);
  if (need > kScratchBytes)
    return set_error(AILA_HIP_EINVAL,
                     "gqa_decode_noalloc: B*Hq = %d heads of D = %d need %zu bytes of split records, above the "
                     "static %zu-byte scratch; use aila_hip_gqa_decode with a workspace",
                     B * Hq, D, need, kScratchBytes);
  float* ws = scratch_for_current_device();
  if (!ws) return AILA_HIP_ELAUNCH;
  // As many records per (sequence, head) as the scratch holds (capped at
  // the split limit); no record needs clearing: the merge reads only the
  // splits that hold rows of the sequence, and each of those is written by
  // its split workgroup in the same call.
  return gqa_decode_impl(q, k_cache, v_cache, out, ws, kScratchBytes, B, Hq, Hkv, D, max_seq, cached_len, seq_lens,
                         0, nullptr, nullptr, static_cast<hipStream_t>(stream));
}

extern "C" int aila_hip_gqa_decode_append(const void* q, const void* k_new, const void* v_new, void* k_cache,
                                          void* v_cache, void* out, void* workspace, size_t workspace_bytes,
                                          int B, int Hq, int Hkv, int D, int max_seq, int pos,
                                          const int* positions, void* stream) {
  using namespace aila;
  AILA_REQUIRE(k_new && v_new, "gqa_decode_append: null k_new/v_new");
  AILA_REQUIRE(pos >= 0 && pos < max_seq, "gqa_decode_append: pos=%d outside [0, max_seq=%d)", pos, max_seq);
  return gqa_decode_impl(q, k_cache, v_cache, out, workspace, workspace_bytes, B, Hq, Hkv, D, max_seq, pos + 1,
                         positions, 1, k_new, v_new, static_cast<hipStream_t>(stream));
}

extern "C" int aila_hip_gqa_decode_prepare_append(const void* q_in, int packed_gate, void* gate_out,
                                                  const void* k_new, const void* v_new, const void* q_norm_w,
                                                  const void* k_norm_w, void* k_cache, void* v_cache, void* out,
                                                  void* workspace, size_t workspace_bytes, int B, int Hq, int Hkv,
                                                  int D, int max_seq, int rotary_dim, float theta, float eps,
                                                  int pos, const int* positions,
                                                  const aila_hip_rope_pos* rope_pos, void* stream) {
  using namespace aila;
  AILA_REQUIRE(k_new && v_new, "gqa_decode_prepare_append: null k_new/v_new");
  AILA_REQUIRE(packed_gate >= 0 && packed_gate <= 2, "gqa_decode_prepare_append: packed_gate=%d not 0, 1 or 2",
               packed_gate);
  AILA_REQUIRE(packed_gate != 1 || gate_out, "gqa_decode_prepare_append: packed q|gate (1) needs gate_out");
  AILA_REQUIRE(pos >= 0 && pos < max_seq, "gqa_decode_prepare_append: pos=%d outside [0, max_seq=%d)", pos,
               max_seq);
  AILA_REQUIRE(theta > 0.f && eps >= 0.f, "gqa_decode_prepare_append: bad theta/eps");
  int rot = std::max(2, std::min(D, rotary_dim));
  if (rot & 1) --rot;
  PrepArgs pa{};
  pa.q_stride = packed_gate ? 2 * D : D;
  pa.qn_w = static_cast<const bf16*>(q_norm_w);
  pa.kn_w = static_cast<const bf16*>(k_norm_w);
  pa.gate_out = packed_gate == 1 ? static_cast<bf16*>(gate_out) : nullptr;
  pa.apply_gate = packed_gate == 2;
  pa.rot = rot;
  pa.freq = rope_freq_table(theta, rot);
  pa.eps = eps;
  if (int rc = load_rope_pos(rope_pos, &pa.rope, "gqa_decode_prepare_append")) return rc;
  return gqa_decode_impl(q_in, k_cache, v_cache, out, workspace, workspace_bytes, B, Hq, Hkv, D, max_seq, pos + 1,
                         positions, 1, k_new, v_new, static_cast<hipStream_t>(stream), &pa);
}

namespace aila {
namespace {
// One new token per sequence: k_new/v_new [B, Hkv, D] -> cache row pos
// (or positions[b]) of [B, Hkv, max_seq, D]. One 16-byte chunk per thread.
__global__ void kv_append_kernel(const u32x4* __restrict__ kn, const u32x4* __restrict__ vn,
                                 bf16* __restrict__ kc, bf16* __restrict__ vc, int B, int Hkv,
                                 int D, int max_seq, int pos, const int* __restrict__ positions) {
  const int chunks = D / 8;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * Hkv * chunks) return;
  const int b = i / (Hkv * chunks);
  const int h = (i / chunks) % Hkv;
  const int c = i % chunks;
  const int p = positions ? positions[b] : pos;
  if (p < 0 || p >= max_seq) return;
  const size_t dst = ((static_cast<size_t>(b) * Hkv + h) * max_seq + p) * D + c * 8;
  *reinterpret_cast<u32x4*>(kc + dst) = kn[i];
  *reinterpret_cast<u32x4*>(vc + dst) = vn[i];
}
}  // namespace
}  // namespace aila

extern "C" int aila_hip_kv_append(const void* k_new, const void* v_new, void* k_cache,
                                  void* v_cache, int B, int Hkv, int D, int max_seq, int pos,
                                  const int* positions, void* stream) {
  using namespace aila;
  AILA_REQUIRE(k_new && v_new && k_cache && v_cache, "kv_append: null pointer");
  AILA_REQUIRE(B > 0 && Hkv > 0 && D > 0 && D % 8 == 0, "kv_append: bad shape (B=%d Hkv=%d D=%d)", B, Hkv, D);
  AILA_REQUIRE(positions || (pos >= 0 && pos < max_seq), "kv_append: pos=%d outside [0, max_seq=%d)", pos, max_seq);
  const int n = B * Hkv * (D / 8);
  hipLaunchKernelGGL(kv_append_kernel, dim3((n + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(k_new), static_cast<const u32x4*>(v_new),
                     static_cast<bf16*>(k_cache), static_cast<bf16*>(v_cache), B, Hkv, D, max_seq, pos,
                     positions);
  return check_launch("kv_append");
}

namespace aila {
namespace {
// One new token per sequence into its page: row positions[b] of sequence b
// is row positions[b] % page_size of page table[b * max_pages +
// positions[b] / page_size]. One 16-byte chunk per thread.
__global__ void kv_append_paged_kernel(const u32x4* __restrict__ kn, const u32x4* __restrict__ vn,
                                       bf16* __restrict__ kp, bf16* __restrict__ vp, int B, int Hkv, int D,
                                       int page_size, const int* __restrict__ table, int max_pages,
                                       const int* __restrict__ positions) {
  const int chunks = D / 8;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * Hkv * chunks) return;
  const int b = i / (Hkv * chunks);
  const int h = (i / chunks) % Hkv;
  const int c = i % chunks;
  const int p = positions[b];
  if (p < 0 || p >= max_pages * page_size) return;
  const int page = table[b * max_pages + p / page_size];
  const size_t dst = ((static_cast<size_t>(page) * Hkv + h) * page_size + p % page_size) * D + c * 8;
  *reinterpret_cast<u32x4*>(kp + dst) = kn[i];
  *reinterpret_cast<u32x4*>(vp + dst) = vn[i];
}
}  // namespace
}  // namespace aila

extern "C" int aila_hip_kv_append_paged(const void* k_new, const void* v_new, void* k_pages, void* v_pages, int B,
                                        int Hkv, int D, int page_size, const int* block_table, int max_pages,
                                        const int* positions, void* stream) {
  using namespace aila;
  AILA_REQUIRE(k_new && v_new && k_pages && v_pages && block_table && positions, "kv_append_paged: null pointer");
  AILA_REQUIRE(B > 0 && Hkv > 0 && D > 0 && D % 8 == 0 && page_size > 0 && max_pages > 0,
               "kv_append_paged: bad shape (B=%d Hkv=%d D=%d page_size=%d max_pages=%d)", B, Hkv, D, page_size,
               max_pages);
  // the same row-range cap as the paged decode (int row arithmetic)
  AILA_REQUIRE(static_cast<long>(max_pages) * page_size <= (1L << 30),
               "kv_append_paged: max_pages * page_size = %ld rows exceeds 2^30", static_cast<long>(max_pages) * page_size);
  // rows move as 16-byte vectors
  AILA_REQUIRE(reinterpret_cast<uintptr_t>(k_new) % 16 == 0 && reinterpret_cast<uintptr_t>(v_new) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(k_pages) % 16 == 0 && reinterpret_cast<uintptr_t>(v_pages) % 16 == 0,
               "kv_append_paged: k_new, v_new, k_pages and v_pages must be 16-byte aligned");
  const int n = B * Hkv * (D / 8);
  hipLaunchKernelGGL(kv_append_paged_kernel, dim3((n + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(k_new), static_cast<const u32x4*>(v_new), static_cast<bf16*>(k_pages),
                     static_cast<bf16*>(v_pages), B, Hkv, D, page_size, block_table, max_pages, positions);
  return check_launch("kv_append_paged");
}

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

__device__ __forceinline__ int vslot(int k) {
  // key k (0..BN-1) -> column in the V^T tile
  return (k & ~31) | (((k & 15) >> 2) << 3) | (((k >> 4) & 1) << 2) | (k & 3);
}

template <int D, int RPW, int BN>
struct PrefillCfg {
  static constexpr int BM = kWaves * RPW;
  static constexpr int QT = RPW / 16;     // 16-row query tiles per wave
  static constexpr int KS = D / 32;       // MFMA k-steps over D (S^T)
  static constexpr int DT = D / 16;       // 16-row d tiles (O^T)
  static constexpr int KT = BN / 16;      // 16-key tiles per block
  static constexpr int PS = BN / 32;      // 32-key MFMA steps (O^T)
  static constexpr int KP = D + 8;        // K tile pitch (bf16 elements)
  static constexpr int VP = BN + 8;       // V^T tile pitch
  static constexpr int KCH = BN * D / 8 / kThreads;        // 16B K chunks / thread
  static constexpr int VU = (BN / 4) * (D / 8);            // 4-key x 8-d V units
  static constexpr int VUT = (VU + kThreads - 1) / kThreads;
  static_assert(BN % 32 == 0 && D % 32 == 0 && RPW % 16 == 0, "tile");
  static_assert((BN * D / 8) % kThreads == 0, "K chunks");
};

template <int D, int RPW, int BN>
__global__ __launch_bounds__(kThreads, 2) void gqa_prefill_kernel(
    const bf16* __restrict__ q, int q_row_stride, const bf16* __restrict__ k,
    const bf16* __restrict__ v, int kv_row_stride, long kv_head_stride,
    bf16* __restrict__ out, int o_row_stride, int S, int start_pos, int Hkv,
    int G, float scale_log2, bf16* __restrict__ k_cache,
    bf16* __restrict__ v_cache, int cache_pos, int max_seq) {
  using C = PrefillCfg<D, RPW, BN>;
  __shared__ __attribute__((aligned(16))) bf16 sK[2][BN * C::KP];
  __shared__ __attribute__((aligned(16))) bf16 sV[2][D * C::VP];

  const int nqb = (S + C::BM - 1) / C::BM;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x);   // heavy blocks first
  const int h = blockIdx.y;
  const int kvh = h / G;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int m16 = lane & 15, g4 = lane >> 4;
  const int q0 = qb * C::BM;
  const int q_hi = min(q0 + C::BM, S) - 1;
  const int kv_len = start_pos + S;
  const int nkb = (start_pos + q_hi) / BN + 1;
  const bf16* Kh = k + kvh * kv_head_stride;
  const bf16* Vh = v + kvh * kv_head_stride;
  const bool write_cache = (k_cache != nullptr) && (h % G == 0);

  // ---- Q^T operands (B of S^T), loaded once ------------------------------
  bf16x8_t qb_op[C::QT][C::KS];
#pragma unroll
  for (int qt = 0; qt < C::QT; ++qt) {
    const int row = min(q0 + wave * RPW + qt * 16 + m16, S - 1);
    const bf16* qr = q + static_cast<size_t>(row) * q_row_stride + h * D + g4 * 8;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) qb_op[qt][ks] = as_bf16x8(ld16(qr + ks * 32));
  }

  // ---- global -> register staging of one K/V block -----------------------
  u32x4 kreg[C::KCH];
  u32x4 vreg[C::VUT][4];
  auto fetch = [&](int kb) {
    const int key0 = kb * BN;
#pragma unroll
    for (int i = 0; i < C::KCH; ++i) {
      const int c = t + i * kThreads;
      const int r = c / (D / 8), c8 = c % (D / 8);
      const int key = min(key0 + r, kv_len - 1);
      kreg[i] = ld16(Kh + static_cast<size_t>(key) * kv_row_stride + c8 * 8);
    }
#pragma unroll
    for (int u = 0; u < C::VUT; ++u) {
      const int unit = t + u * kThreads;
      if (unit < C::VU) {
        const int kg = unit / (D / 8), dc = unit % (D / 8);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int key = min(key0 + kg * 4 + j, kv_len - 1);
          vreg[u][j] = ld16(Vh + static_cast<size_t>(key) * kv_row_stride + dc * 8);
        }
      }
    }
  };
  auto stash = [&](int buf, int kb) {
    const int key0 = kb * BN;
#pragma unroll
    for (int i = 0; i < C::KCH; ++i) {
      const int c = t + i * kThreads;
      const int r = c / (D / 8), c8 = c % (D / 8);
      *reinterpret_cast<u32x4*>(&sK[buf][r * C::KP + c8 * 8]) = kreg[i];
      if (write_cache) {
        const int key = key0 + r;
        if (key >= q0 && key <= q_hi)
          *reinterpret_cast<u32x4*>(k_cache + (static_cast<size_t>(kvh) * max_seq + cache_pos + key) * D + c8 * 8) = kreg[i];
      }
    }
#pragma unroll
    for (int u = 0; u < C::VUT; ++u) {
      const int unit = t + u * kThreads;
      if (unit < C::VU) {
        const int kg = unit / (D / 8), dc = unit % (D / 8);
        // transpose 4 keys x 8 d into 8 rows of V^T (4 contiguous slots)
        const int col = vslot(kg * 4);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int w = e >> 1;
          const bool hi = e & 1;
          uint32_t x0 = hi ? (vreg[u][0][w] >> 16) : (vreg[u][0][w] & 0xffffu);
          uint32_t x1 = hi ? (vreg[u][1][w] >> 16) : (vreg[u][1][w] & 0xffffu);
          uint32_t x2 = hi ? (vreg[u][2][w] >> 16) : (vreg[u][2][w] & 0xffffu);
          uint32_t x3 = hi ? (vreg[u][3][w] >> 16) : (vreg[u][3][w] & 0xffffu);
          u32x2 pk = {x0 | (x1 << 16), x2 | (x3 << 16)};
          *reinterpret_cast<u32x2*>(&sV[buf][(dc * 8 + e) * C::VP + col]) = pk;
        }
        if (write_cache) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int key = key0 + kg * 4 + j;
            if (key >= q0 && key <= q_hi)
              *reinterpret_cast<u32x4*>(v_cache + (static_cast<size_t>(kvh) * max_seq + cache_pos + key) * D + dc * 8) = vreg[u][j];
          }
        }
      }
    }
  };

  f32x4 o_acc[C::DT][C::QT];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
    for (int qt = 0; qt < C::QT; ++qt) o_acc[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[C::QT], l_run[C::QT];
#pragma unroll
  for (int qt = 0; qt < C::QT; ++qt) {
    m_run[qt] = -INFINITY;
    l_run[qt] = 0.f;
  }
  int qpos[C::QT];
#pragma unroll
  for (int qt = 0; qt < C::QT; ++qt) qpos[qt] = start_pos + q0 + wave * RPW + qt * 16 + m16;
  const int wave_qmin = start_pos + q0 + wave * RPW;

  fetch(0);
  stash(0, 0);
  __syncthreads();

  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    if (kb + 1 < nkb) fetch(kb + 1);
    const int key0 = kb * BN;
    // A wave whose rows all precede this block's first key skips it.
    if (key0 <= wave_qmin + RPW - 1) {
      // ---- S^T = K Q^T -----------------------------------------------------
      f32x4 st[C::KT][C::QT];
#pragma unroll
      for (int kt = 0; kt < C::KT; ++kt)
#pragma unroll
        for (int qt = 0; qt < C::QT; ++qt) st[kt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks) {
#pragma unroll
        for (int kt = 0; kt < C::KT; ++kt) {
          const bf16x8_t a = as_bf16x8(
              *reinterpret_cast<const u32x4*>(&sK[buf][(kt * 16 + m16) * C::KP + ks * 32 + g4 * 8]));
#pragma unroll
          for (int qt = 0; qt < C::QT; ++qt) st[kt][qt] = mfma16x16x32(a, qb_op[qt][ks], st[kt][qt]);
        }
      }
      // ---- mask, online softmax ------------------------------------------
      const bool need_mask = (key0 + BN - 1 > wave_qmin);
      float alpha[C::QT];
#pragma unroll
      for (int qt = 0; qt < C::QT; ++qt) {
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < C::KT; ++kt) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float s = st[kt][qt][j] * scale_log2;
            if (need_mask && (key0 + kt * 16 + g4 * 4 + j > qpos[qt])) s = -INFINITY;
            st[kt][qt][j] = s;
            mx = fmaxf(mx, s);
          }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m_run[qt], mx);
        alpha[qt] = (m_run[qt] == -INFINITY) ? 0.f : fast_exp2(m_run[qt] - mn);
        m_run[qt] = mn;
        l_run[qt] *= alpha[qt];
      }
      // P^T operands: step s2 covers keys 32*s2 + {4g..4g+3, 16+4g..16+4g+3}
      bf16x8_t pb[C::PS][C::QT];
#pragma unroll
      for (int s2 = 0; s2 < C::PS; ++s2) {
#pragma unroll
        for (int qt = 0; qt < C::QT; ++qt) {
          const float mref = m_run[qt];
          float p[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            p[j] = fast_exp2(st[2 * s2][qt][j] - mref);
            p[4 + j] = fast_exp2(st[2 * s2 + 1][qt][j] - mref);
          }
#pragma unroll
          for (int j = 0; j < 8; ++j) l_run[qt] += p[j];
          u32x4 w = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]),
                     pack_bf16x2(p[4], p[5]), pack_bf16x2(p[6], p[7])};
          pb[s2][qt] = as_bf16x8(w);
        }
      }
      // ---- O^T = alpha O^T + V^T P^T ---------------------------------------
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int qt = 0; qt < C::QT; ++qt) o_acc[dt][qt] *= alpha[qt];
#pragma unroll
      for (int s2 = 0; s2 < C::PS; ++s2) {
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
          const bf16x8_t a = as_bf16x8(
              *reinterpret_cast<const u32x4*>(&sV[buf][(dt * 16 + m16) * C::VP + s2 * 32 + g4 * 8]));
#pragma unroll
          for (int qt = 0; qt < C::QT; ++qt) o_acc[dt][qt] = mfma16x16x32(a, pb[s2][qt], o_acc[dt][qt]);
        }
      }
    }
    if (kb + 1 < nkb) stash(buf ^ 1, kb + 1);
    __syncthreads();
  }

  // ---- epilogue: normalise, bf16, store ----------------------------------
#pragma unroll
  for (int qt = 0; qt < C::QT; ++qt) {
    float l = l_run[qt];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const float inv = 1.0f / l;
    const int row = q0 + wave * RPW + qt * 16 + m16;
    if (row < S) {
      bf16* orow = out + static_cast<size_t>(row) * o_row_stride + h * D + g4 * 4;
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) {
        const f32x4 o = o_acc[dt][qt] * inv;
        u32x2 w = {pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
        *reinterpret_cast<u32x2*>(orow + dt * 16) = w;
      }
    }
  }
}

template <int D, int RPW, int BN>
int launch_prefill(const bf16* q, const bf16* k, const bf16* v, int kv_row_stride,
                   long kv_head_stride, bf16* out, int S, int start_pos, int Hq,
                   int Hkv, bf16* k_cache, bf16* v_cache, int cache_pos, int max_seq,
                   hipStream_t st) {
  using C = PrefillCfg<D, RPW, BN>;
  const int nqb = (S + C::BM - 1) / C::BM;
  const float scale_log2 = kLog2e / sqrtf(static_cast<float>(D));
  hipLaunchKernelGGL((gqa_prefill_kernel<D, RPW, BN>), dim3(nqb, Hq), dim3(kThreads), 0, st,
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

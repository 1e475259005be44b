// Oracle: scalar CPU restatement of Aila's attention hot path.
//
// TEST INFRASTRUCTURE ONLY. Nothing in the product (aila_amd/, include/)
// links, loads or calls this file. It is used by tests/ as the parity
// checker, by __graft_entry__.smoke() as the checker, and by bench.py's
// cpu_baseline leg as the timed CPU baseline ("kind": "port").
//
// Every function restates the reference's algorithm in plain C++ and cites
// the reference file:line it follows (paths relative to the Aila repo root).
// The reference itself is SYCL (icpx + oneDNN) and cannot be built in this
// image, so there is no oracle/_ref build; parity is pinned by the closed
// forms, invariants and fp64 brute force in tests/test_oracle_*.py.
//
// Numeric conventions follow the reference:
//  * bf16 is stored as uint16_t; bf16 -> f32 is exact; f32 -> bf16 is
//    round-to-nearest-even (sycl::ext::oneapi::bfloat16 constructor).
//  * Accumulation is fp32 in the reference's loop order. The reference's
//    sycl::native::exp / group reductions have no pinned bit pattern; we use
//    std::exp and sequential sums, so parity is tolerance based.
//  * `*_f64` functions are fp64 "truth" versions used to judge tolerances.
//
// Layouts (all row-major):
//  * decode q/out        [B, Hq, D]              (reference: [1, Hq*D], B=1)
//  * KV cache            [B, Hkv, max_seq, D]    (KVCache.hpp:9-45 per sequence)
//  * prefill q/out       [S, Hq*D], k/v [S, Hkv*D] (Ops.hpp:271-282)
//  * DeltaNet q,k        [B, T, Hk, dk]; v [B, T, Hv, dv]; a,b [B, T, Hv]
//    state               [B, Hv, dk, dv]  (S[j*dv + i], Qwen35HybridTextBackend.cpp:1751)

#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>
#include <algorithm>
#include <thread>
#include <omp.h>

typedef uint16_t bf16_t;

extern "C" {

// ---------------------------------------------------------------- bf16 ----
float orc_bf16_to_f32(bf16_t h) {
  uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// Round-to-nearest-even, NaN kept quiet (bfloat16(float) semantics).
bf16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
    return static_cast<bf16_t>((u >> 16) | 0x0040u);
  }
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return static_cast<bf16_t>(u >> 16);
}

void orc_f32_to_bf16_array(const float* x, bf16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_bf16(x[i]);
}

void orc_bf16_to_f32_array(const bf16_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_bf16_to_f32(x[i]);
}

int orc_num_threads(void) { return omp_get_max_threads(); }
void orc_set_num_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }

static inline float bf(bf16_t h) { return orc_bf16_to_f32(h); }

// ------------------------------------------------------ GQA decode --------
// attention_decode_baseline, AttentionOps.cpp:73-166: the effective_len
// attended rows map to cache rows t (t < sink_len) and
// tail_start + (t - sink_len) (:109, :160). Contiguous mode is sink_len = 0,
// tail_start = 0, effective_len = cached_len (:611-616).
// One sequence: q/out [Hq, D], cache [Hkv, max_seq, D].
static void decode_baseline_rows(const bf16_t* q, const bf16_t* kc,
                                 const bf16_t* vc, bf16_t* out, int Hq,
                                 int Hkv, int D, int max_seq, int tail_start,
                                 int sink_len, int L) {
  const int heads_per_kv = Hq / Hkv;                     // :85
  const float scale = 1.0f / std::sqrt(static_cast<float>(D));  // :86
#pragma omp parallel for schedule(static)
  for (int h = 0; h < Hq; ++h) {
    const int kvh = h / heads_per_kv;                    // :100
    std::vector<float> qf(D), sc(L > 0 ? L : 1);
    for (int d = 0; d < D; ++d) qf[d] = bf(q[h * D + d]);        // :102-104
    for (int t = 0; t < L; ++t) {                                 // :107-133
      const int ct = t < sink_len ? t : tail_start + (t - sink_len);
      const bf16_t* kr = kc + (static_cast<size_t>(kvh) * max_seq + ct) * D;
      float s = 0.0f;
      for (int d = 0; d < D; ++d) s += qf[d] * bf(kr[d]);
      sc[t] = s * scale;
    }
    float mx = -1e30f;                                            // :136-141
    for (int t = 0; t < L; ++t) mx = std::fmax(mx, sc[t]);
    float sum = 0.0f;                                             // :143-150
    for (int t = 0; t < L; ++t) {
      float e = std::exp(sc[t] - mx);
      sc[t] = e;
      sum += e;
    }
    for (int t = 0; t < L; ++t) sc[t] = sc[t] / sum;              // :152-156
    for (int d = 0; d < D; ++d) {                                 // :158-166
      float acc = 0.0f;
      for (int t = 0; t < L; ++t) {
        const int ct = t < sink_len ? t : tail_start + (t - sink_len);
        acc += sc[t] * bf(vc[(static_cast<size_t>(kvh) * max_seq + ct) * D + d]);
      }
      out[h * D + d] = orc_f32_to_bf16(acc);
    }
  }
}

static void decode_baseline_one(const bf16_t* q, const bf16_t* kc,
                                const bf16_t* vc, bf16_t* out, int Hq,
                                int Hkv, int D, int max_seq, int L) {
  decode_baseline_rows(q, kc, vc, out, Hq, Hkv, D, max_seq, 0, 0, L);
}

void orc_attention_decode_baseline(const bf16_t* q, const bf16_t* kc,
                                   const bf16_t* vc, bf16_t* out, int B,
                                   int Hq, int Hkv, int D, int max_seq,
                                   int cached_len) {
  for (int b = 0; b < B; ++b)
    decode_baseline_one(q + static_cast<size_t>(b) * Hq * D,
                        kc + static_cast<size_t>(b) * Hkv * max_seq * D,
                        vc + static_cast<size_t>(b) * Hkv * max_seq * D,
                        out + static_cast<size_t>(b) * Hq * D, Hq, Hkv, D,
                        max_seq, cached_len);
}

// ops::attention_decode with the decode window knobs (AttentionOps.cpp:
// 533-551 read them from AILA_ATTN_DECODE_WINDOW / _WINDOW_START / _SINK;
// the window plan is :598-616) on the baseline kernel, per sequence of
// lens[b] rows (or cached_len when lens is null). window_start < 0 is the
// reference's default max(512, window).
void orc_attention_decode_window(const bf16_t* q, const bf16_t* kc, const bf16_t* vc, bf16_t* out, int B,
                                 int Hq, int Hkv, int D, int max_seq, int cached_len, const int* lens,
                                 int window, int window_start, int sink) {
  if (window_start < 0) window_start = std::max(512, window);
  for (int b = 0; b < B; ++b) {
    const int L = lens ? lens[b] : cached_len;
    const bool apply_window = window > 0 && L > window_start;   // :598
    int effective_window = L;
    if (apply_window) effective_window = std::min(L, window);
    int tail_start = L - effective_window;
    int sink_len = 0;
    if (apply_window && sink > 0) sink_len = std::min(sink, std::max(0, L - effective_window));
    int effective_len = effective_window + sink_len;
    if (effective_len >= L) {                                    // :612-616
      tail_start = 0;
      sink_len = 0;
      effective_len = L;
    }
    decode_baseline_rows(q + static_cast<size_t>(b) * Hq * D, kc + static_cast<size_t>(b) * Hkv * max_seq * D,
                         vc + static_cast<size_t>(b) * Hkv * max_seq * D, out + static_cast<size_t>(b) * Hq * D, Hq,
                         Hkv, D, max_seq, tail_start, sink_len, effective_len);
  }
}

// attention_decode_exact_head256_partial_merge, AttentionOps.cpp:168-320,
// generalised to any head_dim and tile length. Phase 1 writes per-tile
// records {m, l, acc[D]} (record layout :50-51: [0]=m, [1]=l, [16..]=acc,
// stride 16 + D); phase 2 merges with exp(m_i - M). `partials` may be null;
// when given it must hold B*Hq*ceil(L/tile)*(16+D) floats and receives the
// phase-1 records ([b][h][tile][16+D]).
void orc_attention_decode_splitk(const bf16_t* q, const bf16_t* kc,
                                 const bf16_t* vc, bf16_t* out, int B, int Hq,
                                 int Hkv, int D, int max_seq, int L, int tile,
                                 float* partials) {
  const int heads_per_kv = Hq / Hkv;
  const float scale = 1.0f / std::sqrt(static_cast<float>(D));
  const int ntiles = (L + tile - 1) / tile;
  const int stride = 16 + D;
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b) {
    for (int h = 0; h < Hq; ++h) {
      const int kvh = h / heads_per_kv;
      const bf16_t* kbase = kc + (static_cast<size_t>(b) * Hkv + kvh) * max_seq * D;
      const bf16_t* vbase = vc + (static_cast<size_t>(b) * Hkv + kvh) * max_seq * D;
      std::vector<float> qf(D), logits(tile), rec(static_cast<size_t>(ntiles) * stride);
      for (int d = 0; d < D; ++d) qf[d] = bf(q[(static_cast<size_t>(b) * Hq + h) * D + d]);
      for (int ti = 0; ti < ntiles; ++ti) {                     // :193-272
        const int t0 = ti * tile;
        const int tl = std::min(tile, L - t0);
        float tmax = -1e30f;
        for (int i = 0; i < tl; ++i) {
          const bf16_t* kr = kbase + static_cast<size_t>(t0 + i) * D;
          float s = 0.0f;
          for (int d = 0; d < D; ++d) s += qf[d] * bf(kr[d]);
          logits[i] = s * scale;
          tmax = std::fmax(tmax, logits[i]);
        }
        float tsum = 0.0f;
        for (int i = 0; i < tl; ++i) {
          logits[i] = std::exp(logits[i] - tmax);
          tsum += logits[i];
        }
        float* r = rec.data() + static_cast<size_t>(ti) * stride;
        std::fill(r, r + stride, 0.0f);
        r[0] = tmax;
        r[1] = tsum;
        for (int d = 0; d < D; ++d) {
          float acc = 0.0f;
          for (int i = 0; i < tl; ++i)
            acc += logits[i] * bf(vbase[static_cast<size_t>(t0 + i) * D + d]);
          r[16 + d] = acc;
        }
      }
      // Phase 2 merge, :276-319.
      float gmax = -1e30f;
      for (int ti = 0; ti < ntiles; ++ti) gmax = std::fmax(gmax, rec[static_cast<size_t>(ti) * stride]);
      std::vector<float> fac(ntiles);
      float sum = 0.0f;
      for (int ti = 0; ti < ntiles; ++ti) {
        fac[ti] = std::exp(rec[static_cast<size_t>(ti) * stride] - gmax);
        sum += fac[ti] * rec[static_cast<size_t>(ti) * stride + 1];
      }
      const float inv = 1.0f / sum;
      for (int d = 0; d < D; ++d) {
        float acc = 0.0f;
        for (int ti = 0; ti < ntiles; ++ti) acc += fac[ti] * rec[static_cast<size_t>(ti) * stride + 16 + d];
        out[(static_cast<size_t>(b) * Hq + h) * D + d] = orc_f32_to_bf16(acc * inv);
      }
      if (partials) {
        std::memcpy(partials + (static_cast<size_t>(b) * Hq + h) * ntiles * stride,
                    rec.data(), rec.size() * sizeof(float));
      }
    }
  }
}

// ----------------------------------------------------- GQA prefill --------
// Naive 3-pass causal prefill, AttentionOps.cpp:769-841: scores with the
// causal mask, row softmax with precise exp (:815), then P.V; bf16 output.
// q [S, Hq*D], k/v [S, Hkv*D] token-major.
void orc_attention_prefill_naive(const bf16_t* q, const bf16_t* k,
                                 const bf16_t* v, bf16_t* out, int S, int Hq,
                                 int Hkv, int D) {
  const int hpk = Hq / Hkv;
  const float scale = 1.0f / std::sqrt(static_cast<float>(D));
  const int qt = Hq * D, kt = Hkv * D;
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
  for (int h = 0; h < Hq; ++h) {
    for (int qi = 0; qi < S; ++qi) {
      const int kvh = h / hpk;
      std::vector<float> row(qi + 1);
      for (int ki = 0; ki <= qi; ++ki) {                          // :784-797
        float dot = 0.0f;
        for (int d = 0; d < D; ++d)
          dot += bf(q[static_cast<size_t>(qi) * qt + h * D + d]) *
                 bf(k[static_cast<size_t>(ki) * kt + kvh * D + d]);
        row[ki] = dot * scale;
      }
      float mx = -1e30f;                                          // :807-820
      for (int ki = 0; ki <= qi; ++ki) mx = std::fmax(mx, row[ki]);
      float sum = 0.0f;
      for (int ki = 0; ki <= qi; ++ki) {
        row[ki] = std::exp(row[ki] - mx);
        sum += row[ki];
      }
      for (int ki = 0; ki <= qi; ++ki) row[ki] /= sum;
      for (int d = 0; d < D; ++d) {                               // :827-840
        float acc = 0.0f;
        for (int t = 0; t <= qi; ++t)
          acc += row[t] * bf(v[static_cast<size_t>(t) * kt + kvh * D + d]);
        out[static_cast<size_t>(qi) * qt + h * D + d] = orc_f32_to_bf16(acc);
      }
    }
  }
}

// Online-softmax causal prefill over key tiles, AttentionOps.cpp:652-767
// (the exact-256 branch), generalised to any D. Keys of tile j are merged
// with alpha = exp(m_prev - m_new), beta = exp(m_tile - m_new) (:731-742).
// When `kc` is non-null the keys come from a cache [Hkv, max_seq, D] and
// query i sits at position start_pos + i (attention_prefill_cached
// :2315-2440); otherwise k/v are token-major [S, Hkv*D] and start_pos = 0.
static void prefill_online_impl(const bf16_t* q, const bf16_t* k,
                                const bf16_t* v, bf16_t* out, int S,
                                int start_pos, int Hq, int Hkv, int D,
                                int max_seq, bool from_cache, int tile) {
  const int hpk = Hq / Hkv;
  const float scale = 1.0f / std::sqrt(static_cast<float>(D));
  const int qt = Hq * D, kt = Hkv * D;
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
  for (int h = 0; h < Hq; ++h) {
    for (int qi = 0; qi < S; ++qi) {
      const int kvh = h / hpk;
      const int q_end = start_pos + qi;
      auto krow = [&](int t) {
        return from_cache ? k + (static_cast<size_t>(kvh) * max_seq + t) * D
                          : k + static_cast<size_t>(t) * kt + kvh * D;
      };
      auto vrow = [&](int t) {
        return from_cache ? v + (static_cast<size_t>(kvh) * max_seq + t) * D
                          : v + static_cast<size_t>(t) * kt + kvh * D;
      };
      std::vector<float> qf(D), acc(D, 0.0f), sc(tile);
      for (int d = 0; d < D; ++d) qf[d] = bf(q[static_cast<size_t>(qi) * qt + h * D + d]);
      float m = -1e30f, l = 0.0f;
      for (int t0 = 0; t0 <= q_end; t0 += tile) {
        const int tl = std::min(tile, q_end + 1 - t0);
        float tmax = -1e30f;
        for (int i = 0; i < tl; ++i) {
          const bf16_t* kr = krow(t0 + i);
          float s = 0.0f;
          for (int d = 0; d < D; ++d) s += qf[d] * bf(kr[d]);
          sc[i] = s * scale;
          tmax = std::fmax(tmax, sc[i]);
        }
        float tsum = 0.0f;
        for (int i = 0; i < tl; ++i) {
          sc[i] = std::exp(sc[i] - tmax);
          tsum += sc[i];
        }
        const float mn = std::fmax(m, tmax);
        const float al = std::exp(m - mn), be = std::exp(tmax - mn);
        m = mn;
        l = al * l + be * tsum;
        for (int d = 0; d < D; ++d) {
          float ta = 0.0f;
          for (int i = 0; i < tl; ++i) ta += sc[i] * bf(vrow(t0 + i)[d]);
          acc[d] = al * acc[d] + be * ta;
        }
      }
      const float inv = 1.0f / l;
      for (int d = 0; d < D; ++d)
        out[static_cast<size_t>(qi) * qt + h * D + d] = orc_f32_to_bf16(acc[d] * inv);
    }
  }
}

void orc_attention_prefill_online(const bf16_t* q, const bf16_t* k,
                                  const bf16_t* v, bf16_t* out, int S, int Hq,
                                  int Hkv, int D, int tile) {
  prefill_online_impl(q, k, v, out, S, 0, Hq, Hkv, D, 0, false, tile);
}

// attention_prefill_cached, AttentionOps.cpp:2308-2507: queries at
// positions start_pos + i attend keys [0, start_pos + i] of the cache.
// online != 0 follows the tiled branch (:2315-2440), else the naive branch
// (:2442-2506).
void orc_attention_prefill_cached(const bf16_t* q, const bf16_t* kc,
                                  const bf16_t* vc, bf16_t* out, int S,
                                  int start_pos, int Hq, int Hkv, int D,
                                  int max_seq, int online) {
  if (online) {
    prefill_online_impl(q, kc, vc, out, S, start_pos, Hq, Hkv, D, max_seq, true, 128);
    return;
  }
  const int hpk = Hq / Hkv;
  const float scale = 1.0f / std::sqrt(static_cast<float>(D));
  const int qt = Hq * D;
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
  for (int h = 0; h < Hq; ++h) {
    for (int qi = 0; qi < S; ++qi) {
      const int kvh = h / hpk;
      const int q_end = start_pos + qi;
      std::vector<float> row(q_end + 1);
      for (int ki = 0; ki <= q_end; ++ki) {
        float dot = 0.0f;
        for (int d = 0; d < D; ++d)
          dot += bf(q[static_cast<size_t>(qi) * qt + h * D + d]) *
                 bf(kc[(static_cast<size_t>(kvh) * max_seq + ki) * D + d]);
        row[ki] = dot * scale;
      }
      float mx = -1e30f;
      for (int ki = 0; ki <= q_end; ++ki) mx = std::fmax(mx, row[ki]);
      float sum = 0.0f;
      for (int ki = 0; ki <= q_end; ++ki) {
        row[ki] = std::exp(row[ki] - mx);
        sum += row[ki];
      }
      for (int ki = 0; ki <= q_end; ++ki) row[ki] /= sum;
      for (int d = 0; d < D; ++d) {
        float acc = 0.0f;
        for (int t = 0; t <= q_end; ++t)
          acc += row[t] * bf(vc[(static_cast<size_t>(kvh) * max_seq + t) * D + d]);
        out[static_cast<size_t>(qi) * qt + h * D + d] = orc_f32_to_bf16(acc);
      }
    }
  }
}

// copy_to_cache, AttentionOps.cpp:2513-2532: [S, H*D] -> [H, max_seq, D] at
// row start_pos.
void orc_copy_to_cache(const bf16_t* src, bf16_t* cache, int S, int start_pos,
                       int H, int D, int max_seq) {
  for (int s = 0; s < S; ++s)
    for (int f = 0; f < H * D; ++f) {
      const int h = f / D, d = f % D;
      cache[(static_cast<size_t>(h) * max_seq + start_pos + s) * D + d] =
          src[static_cast<size_t>(s) * H * D + f];
    }
}

// fp64 truth: causal attention of S queries at positions start_pos + i over
// a cache [Hkv, max_seq, D] (one sequence). Output fp64 [S, Hq, D].
void orc_attention_f64(const bf16_t* q, const bf16_t* kc, const bf16_t* vc,
                       double* out, int S, int start_pos, int Hq, int Hkv,
                       int D, int max_seq) {
  const int hpk = Hq / Hkv;
  const double scale = 1.0 / std::sqrt(static_cast<double>(D));
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
  for (int h = 0; h < Hq; ++h) {
    for (int qi = 0; qi < S; ++qi) {
      const int kvh = h / hpk;
      const int n = start_pos + qi + 1;
      std::vector<double> p(n);
      double mx = -1e300;
      for (int t = 0; t < n; ++t) {
        double s = 0.0;
        for (int d = 0; d < D; ++d)
          s += static_cast<double>(bf(q[(static_cast<size_t>(qi) * Hq + h) * D + d])) *
               bf(kc[(static_cast<size_t>(kvh) * max_seq + t) * D + d]);
        p[t] = s * scale;
        mx = std::max(mx, p[t]);
      }
      double sum = 0.0;
      for (int t = 0; t < n; ++t) {
        p[t] = std::exp(p[t] - mx);
        sum += p[t];
      }
      for (int d = 0; d < D; ++d) {
        double acc = 0.0;
        for (int t = 0; t < n; ++t)
          acc += p[t] * bf(vc[(static_cast<size_t>(kvh) * max_seq + t) * D + d]);
        out[(static_cast<size_t>(qi) * Hq + h) * D + d] = acc / sum;
      }
    }
  }
}

// ---------------------------------------------- QK-norm and RoPE ---------
// head_rms_norm, NormOps.cpp:277-321: per (row, head) x <- bf16(x / rms * w),
// rms = sqrt(mean(x^2) + eps). Weight is bf16 when w_bf16 != null else f32.
void orc_head_rms_norm(bf16_t* x, const bf16_t* w_bf16, const float* w_f32,
                       float eps, int S, int H, int D) {
  for (int g = 0; g < S * H; ++g) {
    bf16_t* r = x + static_cast<size_t>(g) * D;
    float ss = 0.0f;
    for (int d = 0; d < D; ++d) ss += bf(r[d]) * bf(r[d]);
    const float rms = std::sqrt(ss / static_cast<float>(D) + eps);
    for (int d = 0; d < D; ++d) {
      const float w = w_bf16 ? bf(w_bf16[d]) : (w_f32 ? w_f32[d] : 1.0f);
      r[d] = orc_f32_to_bf16(bf(r[d]) / rms * w);
    }
  }
}

// apply_rope_partial, ElementwiseOps.cpp:33-103: NeoX half-split rotation of
// the first `rot` dims of every head for the token at global position
// start_pos + s; freq = 1 / theta^(2d/rot); q and k rounded to bf16. The
// rotary position is the global position, shifted by text_pos_delta past
// prompt_pos_len (:54-58); with `interleaved` and all three streams, pair d
// takes the h stream when d%3 == 1 and d/3 < sec_h, the w stream when
// d%3 == 2 and d/3 < sec_w, else the t stream, each read at the global
// position inside the prompt and equal to the shifted scalar past it
// (:60-78). sec_t is unused, as in the reference. The k rows rotate in the
// same pass for heads h < Hkv of the q-head loop.
void orc_apply_rope_partial(bf16_t* q, bf16_t* k, int S, int start_pos, int Hq, int Hkv, int D,
                            int rotary_dim, float theta, int interleaved, const int* pos_t,
                            const int* pos_h, const int* pos_w, int prompt_pos_len,
                            int text_pos_delta, int sec_t, int sec_h, int sec_w) {
  (void)sec_t;
  int rot = std::max(2, std::min(D, rotary_dim));
  if (rot & 1) --rot;
  const int half = rot / 2;
  for (int s = 0; s < S; ++s)
    for (int h = 0; h < Hq; ++h)
      for (int d = 0; d < half; ++d) {
        const int global_pos = start_pos + s;
        int pos_scalar = global_pos;
        if (global_pos >= prompt_pos_len) pos_scalar = global_pos + text_pos_delta;
        float pos = static_cast<float>(pos_scalar);
        if (interleaved && pos_t && pos_h && pos_w) {
          int stream = 0;
          if ((d % 3) == 1 && (d / 3) < sec_h) stream = 1;
          else if ((d % 3) == 2 && (d / 3) < sec_w) stream = 2;
          const bool in_prompt = global_pos < prompt_pos_len;
          const int t_val = in_prompt ? pos_t[global_pos] : pos_scalar;
          const int h_val = in_prompt ? pos_h[global_pos] : pos_scalar;
          const int w_val = in_prompt ? pos_w[global_pos] : pos_scalar;
          pos = static_cast<float>(stream == 1 ? h_val : stream == 2 ? w_val : t_val);
        }
        const float freq = 1.0f / std::pow(theta, (2.0f * d) / static_cast<float>(rot));
        const float ang = pos * freq;
        const float c = std::cos(ang), sn = std::sin(ang);
        bf16_t* qr = q + (static_cast<size_t>(s) * Hq + h) * D;
        const float q0 = bf(qr[d]), q1 = bf(qr[d + half]);
        qr[d] = orc_f32_to_bf16(q0 * c - q1 * sn);
        qr[d + half] = orc_f32_to_bf16(q1 * c + q0 * sn);
        if (h < Hkv) {
          bf16_t* kr = k + (static_cast<size_t>(s) * Hkv + h) * D;
          const float k0 = bf(kr[d]), k1 = bf(kr[d + half]);
          kr[d] = orc_f32_to_bf16(k0 * c - k1 * sn);
          kr[d + half] = orc_f32_to_bf16(k1 * c + k0 * sn);
        }
      }
}

// Text positions only (no shift, no streams): position start_pos + s.
void orc_apply_rope(bf16_t* q, bf16_t* k, int S, int start_pos, int Hq,
                    int Hkv, int D, int rotary_dim, float theta) {
  orc_apply_rope_partial(q, k, S, start_pos, Hq, Hkv, D, rotary_dim, theta, 0, nullptr, nullptr, nullptr, 0, 0,
                         0, 0, 0);
}

// decode_prepare_qkv, ElementwiseOps.cpp:105-216 (full rotary, one token):
// q,k per-head RMSNorm (bf16 round), RoPE at start_pos (bf16 round), then
// k,v appended to the cache row start_pos. Angle = start_pos * freq[d] with
// freq[d] = 1 / theta^(2d/D) (the backend's rope_freq table).
void orc_decode_prepare_qkv(bf16_t* q, bf16_t* k, const bf16_t* v,
                            const bf16_t* qn_w, const bf16_t* kn_w,
                            bf16_t* kc, bf16_t* vc, int start_pos, int Hq,
                            int Hkv, int D, float eps, float theta,
                            int max_seq) {
  orc_head_rms_norm(q, qn_w, nullptr, eps, 1, Hq, D);
  orc_head_rms_norm(k, kn_w, nullptr, eps, 1, Hkv, D);
  orc_apply_rope(q, k, 1, start_pos, Hq, Hkv, D, D, theta);
  orc_copy_to_cache(k, kc, 1, start_pos, Hkv, D, max_seq);
  orc_copy_to_cache(v, vc, 1, start_pos, Hkv, D, max_seq);
}

// decode_prepare_qkv with the backend's frequency table, as the reference
// computes it (ElementwiseOps.cpp:105-216): per head RMSNorm (bf16 round),
// then pair d of q and k rotated by angle = start_pos * rope_freq[d] over the
// full head (bf16 round), then k, v appended at start_pos. One sequence:
// q [Hq, D], k/v [Hkv, D] (q, k in place), caches [Hkv, max_seq, D].
void orc_decode_prepare_qkv_freq(bf16_t* q, bf16_t* k, const bf16_t* v, const float* rope_freq,
                                 const bf16_t* qn_w, const bf16_t* kn_w, bf16_t* kc, bf16_t* vc, int start_pos,
                                 int Hq, int Hkv, int D, float eps, int max_seq) {
  orc_head_rms_norm(q, qn_w, nullptr, eps, 1, Hq, D);
  orc_head_rms_norm(k, kn_w, nullptr, eps, 1, Hkv, D);
  const int half = D / 2;
  auto rotate = [&](bf16_t* x) {
    for (int d = 0; d < half; ++d) {
      const float angle = static_cast<float>(start_pos) * rope_freq[d];   // :159, :198
      const float c = std::cos(angle), sn = std::sin(angle);
      const float x0 = bf(x[d]), x1 = bf(x[d + half]);
      x[d] = orc_f32_to_bf16(x0 * c - x1 * sn);
      x[d + half] = orc_f32_to_bf16(x1 * c + x0 * sn);
    }
  };
  for (int h = 0; h < Hq; ++h) rotate(q + static_cast<size_t>(h) * D);
  for (int h = 0; h < Hkv; ++h) rotate(k + static_cast<size_t>(h) * D);
  if (kc) {
    orc_copy_to_cache(k, kc, 1, start_pos, Hkv, D, max_seq);
    orc_copy_to_cache(v, vc, 1, start_pos, Hkv, D, max_seq);
  }
}

// decode_prepare_qkv_partial (ElementwiseOps.cpp:555-705) and
// decode_prepare_qgkv_packed_partial (:707-863), batched over B independent
// sequences (the reference runs one): per head, q (the first D of a packed
// [q | gate] head when packed, gate copied through) and k get RMSNorm (bf16
// round) then RoPE over the first `rot` dims for the token at global position
// pos[b] (bf16 round; the rotary_position lambda, :593-617, is
// apply_rope_partial's position rule at that one position); k, v are appended
// to the cache row pos[b] when kc != null.
// q_in [B,Hq,D or 2D]; q_out, gate_out [B,Hq,D]; k (in place), v [B,Hkv,D];
// kc, vc [B,Hkv,max_seq,D]. Rotary positions: sequence b reads its streams
// at pos_t/h/w + b*pos_stride, its prompt length and text delta from
// prompt_lens[b] / deltas[b] when given, else the scalars.
void orc_decode_prepare_rp(const bf16_t* q_in, int packed, bf16_t* q_out, bf16_t* gate_out, bf16_t* k,
                           const bf16_t* v, const bf16_t* qn_w, const bf16_t* kn_w, bf16_t* kc, bf16_t* vc,
                           int B, int Hq, int Hkv, int D, int max_seq, int rotary_dim, float theta,
                           float eps, const int* pos, int interleaved, const int* pos_t, const int* pos_h,
                           const int* pos_w, int pos_stride, int prompt_pos_len, int text_pos_delta,
                           const int* prompt_lens, const int* deltas, int sec_t, int sec_h, int sec_w) {
  const int qs = packed ? 2 * D : D;
  for (int b = 0; b < B; ++b) {
    bf16_t* qo = q_out + static_cast<size_t>(b) * Hq * D;
    for (int h = 0; h < Hq; ++h) {
      const bf16_t* src = q_in + (static_cast<size_t>(b) * Hq + h) * qs;
      for (int d = 0; d < D; ++d) qo[h * D + d] = src[d];
      if (packed)
        for (int d = 0; d < D; ++d) gate_out[(static_cast<size_t>(b) * Hq + h) * D + d] = src[D + d];
    }
    bf16_t* kb = k + static_cast<size_t>(b) * Hkv * D;
    orc_head_rms_norm(qo, qn_w, nullptr, eps, 1, Hq, D);
    orc_head_rms_norm(kb, kn_w, nullptr, eps, 1, Hkv, D);
    const size_t off = static_cast<size_t>(b) * pos_stride;
    orc_apply_rope_partial(qo, kb, 1, pos[b], Hq, Hkv, D, rotary_dim, theta, interleaved,
                           pos_t ? pos_t + off : nullptr, pos_h ? pos_h + off : nullptr,
                           pos_w ? pos_w + off : nullptr, prompt_lens ? prompt_lens[b] : prompt_pos_len,
                           deltas ? deltas[b] : text_pos_delta, sec_t, sec_h, sec_w);
    if (kc) {
      for (int h = 0; h < Hkv; ++h) {
        const size_t row = ((static_cast<size_t>(b) * Hkv + h) * max_seq + pos[b]) * D;
        for (int d = 0; d < D; ++d) {
          kc[row + d] = kb[h * D + d];
          vc[row + d] = v[(static_cast<size_t>(b) * Hkv + h) * D + d];
        }
      }
    }
  }
}

// The same at text positions (rotary position = cache row).
void orc_decode_prepare(const bf16_t* q_in, int packed, bf16_t* q_out, bf16_t* gate_out, bf16_t* k,
                        const bf16_t* v, const bf16_t* qn_w, const bf16_t* kn_w, bf16_t* kc, bf16_t* vc,
                        int B, int Hq, int Hkv, int D, int max_seq, int rotary_dim, float theta,
                        float eps, const int* pos) {
  orc_decode_prepare_rp(q_in, packed, q_out, gate_out, k, v, qn_w, kn_w, kc, vc, B, Hq, Hkv, D, max_seq,
                        rotary_dim, theta, eps, pos, 0, nullptr, nullptr, nullptr, 0, 0, 0, nullptr, nullptr, 0,
                        0, 0);
}

// sigmoid_mul, ElementwiseOps.cpp:519-553: o = bf16(in * 1/(1+e^-g)).
void orc_sigmoid_mul(const bf16_t* in, const bf16_t* g, bf16_t* o, long n) {
  for (long i = 0; i < n; ++i) o[i] = orc_f32_to_bf16(bf(in[i]) * (1.0f / (1.0f + std::exp(-bf(g[i])))));
}

// ------------------------------------------------------- DeltaNet --------
}  // extern "C" (templates below need C++ linkage)
// softplus, Qwen35HybridTextBackend.cpp:128-132.
template <typename R>
static inline R softplus_t(R x) {
  if (x > R(20)) return x;
  if (x < R(-20)) return std::exp(x);
  return std::log1p(std::exp(x));
}

// Key head serving value head hv: contiguous grouping,
// Qwen35HybridTextBackend.cpp:104-118.
static inline int key_head_for(int hv, int Hk, int Hv) {
  if (Hk <= 0 || Hv % Hk != 0) return std::clamp(hv, 0, std::max(0, Hk - 1));
  return std::min(hv / (Hv / Hk), Hk - 1);
}

// Gated delta rule recurrence, following run_linear_delta_host
// (Qwen35HybridTextBackend.cpp:1729-1780) after conv/SiLU:
//   q,k <- x / sqrt(sum x^2 + eps)              (:138-151, when l2norm)
//   beta = sigmoid(b), decay = exp(softplus(a + dt_bias) * -exp(A_log))
//   S *= decay; u = S^T k; d = (v - u) * beta; S += k d^T; o = S^T q * scale
// S is [dk, dv] row-major per (b, hv) (S[j*dv + i]). Inputs bf16
// (q,k [B,T,Hk,dk], v [B,T,Hv,dv], a,b [B,T,Hv]); dt_bias bf16 [Hv] and
// A_log f32 [Hv] may be null (treated as 0). Outputs: o in f32 and/or bf16
// [B,T,Hv,dv] (either may be null). R selects f32 (reference) or f64 (truth).
static inline float ld(bf16_t x) { return bf(x); }
static inline float ld(float x) { return x; }

// In = bf16_t (the op's bf16 inputs) or float (the layer's fp32 conv outputs).
template <typename R, typename In = bf16_t>
static void deltanet_impl(const In* q, const In* k, const In* v,
                          const bf16_t* a, const bf16_t* b,
                          const bf16_t* dt_bias, const float* A_log, R* state,
                          R* out, bf16_t* out_bf16, int B, int T, int Hk,
                          int Hv, int dk, int dv, float eps, float scale,
                          int l2norm) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int bb = 0; bb < B; ++bb) {
    for (int hv = 0; hv < Hv; ++hv) {
      const int hk = key_head_for(hv, Hk, Hv);
      R* S = state + (static_cast<size_t>(bb) * Hv + hv) * dk * dv;
      std::vector<R> qf(dk), kf(dk), u(dv), dd(dv);
      for (int t = 0; t < T; ++t) {
        const size_t bt = static_cast<size_t>(bb) * T + t;
        const In* qr = q + (bt * Hk + hk) * dk;
        const In* kr = k + (bt * Hk + hk) * dk;
        const In* vr = v + (bt * Hv + hv) * dv;
        for (int j = 0; j < dk; ++j) { qf[j] = ld(qr[j]); kf[j] = ld(kr[j]); }
        if (l2norm) {
          R sq = 0, sk = 0;
          for (int j = 0; j < dk; ++j) { sq += qf[j] * qf[j]; sk += kf[j] * kf[j]; }
          const R iq = R(1) / std::sqrt(sq + R(eps));
          const R ik = R(1) / std::sqrt(sk + R(eps));
          for (int j = 0; j < dk; ++j) { qf[j] *= iq; kf[j] *= ik; }
        }
        const R beta = R(1) / (R(1) + std::exp(-static_cast<R>(bf(b[bt * Hv + hv]))));
        const R dtb = dt_bias ? static_cast<R>(bf(dt_bias[hv])) : R(0);
        const R negA = A_log ? -std::exp(static_cast<R>(A_log[hv])) : R(-1);
        const R g = softplus_t<R>(static_cast<R>(bf(a[bt * Hv + hv])) + dtb) * negA;
        const R decay = std::exp(g);
        for (int idx = 0; idx < dk * dv; ++idx) S[idx] *= decay;       // :1749
        for (int i = 0; i < dv; ++i) {                                  // :1751-1758
          R acc = 0;
          for (int j = 0; j < dk; ++j) acc += S[static_cast<size_t>(j) * dv + i] * kf[j];
          u[i] = acc;
          dd[i] = (static_cast<R>(ld(vr[i])) - acc) * beta;
        }
        for (int j = 0; j < dk; ++j) {                                  // :1760-1766
          R* row = S + static_cast<size_t>(j) * dv;
          for (int i = 0; i < dv; ++i) row[i] += kf[j] * dd[i];
        }
        for (int i = 0; i < dv; ++i) {                                  // :1768-1778
          R acc = 0;
          for (int j = 0; j < dk; ++j) acc += S[static_cast<size_t>(j) * dv + i] * qf[j];
          const R o = acc * R(scale);
          const size_t oi = (bt * Hv + hv) * dv + i;
          if (out) out[oi] = o;
          if (out_bf16) out_bf16[oi] = orc_f32_to_bf16(static_cast<float>(o));
        }
      }
    }
  }
}

extern "C" {

void orc_deltanet_recurrent(const bf16_t* q, const bf16_t* k, const bf16_t* v,
                            const bf16_t* a, const bf16_t* b,
                            const bf16_t* dt_bias, const float* A_log,
                            float* state, float* out, bf16_t* out_bf16, int B,
                            int T, int Hk, int Hv, int dk, int dv, float eps,
                            float scale, int l2norm) {
  deltanet_impl<float>(q, k, v, a, b, dt_bias, A_log, state, out, out_bf16, B,
                       T, Hk, Hv, dk, dv, eps, scale, l2norm);
}

// Full Gated DeltaNet layer core, following run_linear_delta_host
// (Qwen35HybridTextBackend.cpp:1640-1798) with the device paths' conv ring
// (:1013-1056 decode, :1376-1411 prefill):
//   conv: per channel c of the [q | k | v] row (conv_ch = 2*Hk*dk + Hv*dv),
//     y = silu(sum_{j<K-1} ring[(head + j) % (K-1)][c] * w[c*K + j]
//              + x[c] * w[c*K + K-1])          (fp32, summed in that order)
//     then ring[head][c] = x[c], head = (head + 1) % (K-1)
//   recurrence on the fp32 conv outputs (deltanet_impl, l2norm on)
//   gate: o <- o / sqrt(mean(o^2) + eps) * norm_w * silu(z)  per value head
//     (head_rms_norm_and_silu_gate, :153-173), rounded to bf16.
// Token rows: qkv at qkv + (b*T + t) * qkv_stride, z likewise with z_stride,
// a and b with ab_stride (so the backend's fused [qkv | z | a | b] row is
// qkv_stride = z_stride = ab_stride = its width). conv_w [conv_ch, K] bf16;
// conv_state [B, K-1, conv_ch] fp32; norm_w [dv] fp32; out [B, T, Hv*dv].
// The caller advances conv_head by T, as the backend does (:1506).
void orc_deltanet_layer(const bf16_t* qkv, int qkv_stride, const bf16_t* z, int z_stride,
                        const bf16_t* a, const bf16_t* b, int ab_stride, const bf16_t* conv_w,
                        float* conv_state, int conv_head, const bf16_t* dt_bias, const float* A_log,
                        const float* norm_w, float* state, bf16_t* out, int B, int T, int Hk, int Hv,
                        int dk, int dv, int K, float eps, float scale) {
  const int qd = Hk * dk, vd = Hv * dv, ch = 2 * qd + vd, R = K - 1;
  const size_t BT = static_cast<size_t>(B) * T;
  std::vector<float> qf(BT * qd), kf(BT * qd), vf(BT * vd), of(BT * vd);
  std::vector<bf16_t> ag(BT * Hv), bg(BT * Hv);
  auto silu = [](float x) { return x / (1.0f + std::exp(-x)); };
  for (int bb = 0; bb < B; ++bb) {
    float* ring = conv_state + static_cast<size_t>(bb) * R * ch;
    int head = R > 0 ? ((conv_head % R) + R) % R : 0;
    for (int t = 0; t < T; ++t) {
      const size_t bt = static_cast<size_t>(bb) * T + t;
      const bf16_t* x = qkv + bt * qkv_stride;
      for (int c = 0; c < ch; ++c) {
        const bf16_t* w = conv_w + static_cast<size_t>(c) * K;
        float acc = 0.0f;
        for (int j = 0; j < R; ++j) acc += ring[static_cast<size_t>((head + j) % R) * ch + c] * bf(w[j]);
        acc += bf(x[c]) * bf(w[R]);
        const float y = silu(acc);
        if (c < qd) qf[bt * qd + c] = y;
        else if (c < 2 * qd) kf[bt * qd + c - qd] = y;
        else vf[bt * vd + c - 2 * qd] = y;
      }
      if (R > 0) {
        for (int c = 0; c < ch; ++c) ring[static_cast<size_t>(head) * ch + c] = bf(x[c]);
        head = (head + 1) % R;
      }
      for (int h = 0; h < Hv; ++h) {
        ag[bt * Hv + h] = a[bt * ab_stride + h];
        bg[bt * Hv + h] = b[bt * ab_stride + h];
      }
    }
  }
  deltanet_impl<float, float>(qf.data(), kf.data(), vf.data(), ag.data(), bg.data(), dt_bias, A_log, state,
                              of.data(), nullptr, B, T, Hk, Hv, dk, dv, eps, scale, 1);
  for (size_t bt = 0; bt < BT; ++bt)
    for (int h = 0; h < Hv; ++h) {
      const float* o = of.data() + (bt * Hv + h) * dv;
      const bf16_t* zg = z + bt * z_stride + static_cast<size_t>(h) * dv;
      float ss = 0.0f;
      for (int i = 0; i < dv; ++i) ss += o[i] * o[i];
      const float inv = 1.0f / std::sqrt(ss / static_cast<float>(dv) + eps);
      for (int i = 0; i < dv; ++i)
        out[(bt * Hv + h) * dv + i] = orc_f32_to_bf16(o[i] * inv * norm_w[i] * silu(bf(zg[i])));
    }
}

void orc_deltanet_recurrent_f64(const bf16_t* q, const bf16_t* k,
                                const bf16_t* v, const bf16_t* a,
                                const bf16_t* b, const bf16_t* dt_bias,
                                const float* A_log, double* state, double* out,
                                int B, int T, int Hk, int Hv, int dk, int dv,
                                float eps, float scale, int l2norm) {
  deltanet_impl<double>(q, k, v, a, b, dt_bias, A_log, state, out, nullptr, B,
                        T, Hk, Hv, dk, dv, eps, scale, l2norm);
}

}  // extern "C"

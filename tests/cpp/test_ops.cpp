// C++ parity test of the ops:: layer (aila_amd/host) on the GPU, checked
// against the CPU oracle (oracle/liboracle.so). Exit code 0 = all passed.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <vector>

#include "Ops.hpp"
#include "aila_hip.h"

extern "C" {
void orc_attention_decode_baseline(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, int, int,
                                   int, int, int, int);
void orc_attention_decode_window(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int,
                                 int, int, const int*, int, int, int);
void orc_attention_prefill_naive(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, int, int,
                                 int, int);
void orc_attention_prefill_cached(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, int, int,
                                  int, int, int, int, int);
void orc_copy_to_cache(const uint16_t*, uint16_t*, int, int, int, int, int);
void orc_deltanet_recurrent(const uint16_t*, const uint16_t*, const uint16_t*, const uint16_t*,
                            const uint16_t*, const uint16_t*, const float*, float*, float*, uint16_t*, int,
                            int, int, int, int, int, float, float, int);
void orc_head_rms_norm(uint16_t*, const uint16_t*, const float*, float, int, int, int);
void orc_apply_rope(uint16_t*, uint16_t*, int, int, int, int, int, int, float);
void orc_decode_prepare_qkv_freq(uint16_t*, uint16_t*, const uint16_t*, const float*, const uint16_t*,
                                 const uint16_t*, uint16_t*, uint16_t*, int, int, int, int, float, int);
void orc_apply_rope_partial(uint16_t*, uint16_t*, int, int, int, int, int, int, float, int, const int*, const int*,
                            const int*, int, int, int, int, int);
void orc_decode_prepare_rp(const uint16_t*, int, uint16_t*, uint16_t*, uint16_t*, const uint16_t*, const uint16_t*,
                           const uint16_t*, uint16_t*, uint16_t*, int, int, int, int, int, int, float, float,
                           const int*, int, const int*, const int*, const int*, int, int, int, const int*,
                           const int*, int, int, int);
void orc_decode_prepare(const uint16_t*, int, uint16_t*, uint16_t*, uint16_t*, const uint16_t*, const uint16_t*,
                        const uint16_t*, uint16_t*, uint16_t*, int, int, int, int, int, int, float, float,
                        const int*);
void orc_decode_prepare_qkv(uint16_t*, uint16_t*, const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*,
                            uint16_t*, int, int, int, int, float, float, int);
void orc_sigmoid_mul(const uint16_t*, const uint16_t*, uint16_t*, long);
void orc_deltanet_layer(const uint16_t*, int, const uint16_t*, int, const uint16_t*, const uint16_t*, int,
                        const uint16_t*, float*, int, const uint16_t*, const float*, const float*, float*, uint16_t*,
                        int, int, int, int, int, int, int, float, float);
uint16_t orc_f32_to_bf16(float);
float orc_bf16_to_f32(uint16_t);
}

using u16v = std::vector<uint16_t>;

static int g_fail = 0;

static uint64_t g_state = 0x1234567ull;
static float nrand() {  // Box-Muller over a 64-bit LCG (test-local inputs)
  auto u = [] {
    g_state = g_state * 6364136223846793005ull + 1442695040888963407ull;
    return ((g_state >> 11) + 0.5) * (1.0 / 9007199254740992.0);
  };
  return static_cast<float>(std::sqrt(-2.0 * std::log(u())) * std::cos(6.283185307179586 * u()));
}
static u16v rand_bf16(size_t n) {
  u16v v(n);
  for (auto& x : v) x = orc_f32_to_bf16(nrand());
  return v;
}
static double relerr(const u16v& a, const u16v& r) {
  double m = 0, d = 0;
  for (size_t i = 0; i < a.size(); ++i) {
    const double x = orc_bf16_to_f32(a[i]), y = orc_bf16_to_f32(r[i]);
    d = std::fmax(d, std::fabs(x - y));
    m = std::fmax(m, std::fabs(y));
  }
  return d / std::fmax(m, 1e-30);
}
static double relerr_f(const std::vector<float>& a, const std::vector<float>& r) {
  double m = 0, d = 0;
  for (size_t i = 0; i < a.size(); ++i) {
    d = std::fmax(d, std::fabs(a[i] - r[i]));
    m = std::fmax(m, std::fabs(r[i]));
  }
  return d / std::fmax(m, 1e-30);
}
static void expect(bool ok, const char* name, double err) {
  std::printf("%-44s %s (err %.3g)\n", name, ok ? "OK" : "FAIL", err);
  if (!ok) ++g_fail;
}
template <typename T>
static Tensor upload(Context& ctx, const std::vector<T>& h, std::vector<int64_t> shape, DType dt) {
  Tensor t = Tensor::allocate(ctx, shape, dt);
  ctx.memcpy_h2d(t.data(), h.data(), h.size() * sizeof(T));
  return t;
}

// The backends' rope_freq table, 1/theta^(2d/head_dim) (Qwen3DenseBackend.cpp:232-236).
static Tensor rope_freq_table(Context& ctx, int D, float theta) {
  std::vector<float> tab(D / 2);
  for (int d = 0; d < D / 2; ++d) tab[d] = 1.0f / std::pow(theta, (2.0f * d) / float(D));
  return upload(ctx, tab, {D / 2}, DType::f32);
}
template <typename T>
static std::vector<T> download(Context& ctx, Tensor& t) {
  std::vector<T> h(t.numel());
  ctx.memcpy_d2h(h.data(), t.data(), h.size() * sizeof(T));
  return h;
}

// A backend-shaped caller: the per-layer attention statements of a dense
// Qwen3 backend (Qwen3DenseBackend.cpp:293-347) use unqualified ops:: calls
// on a global Context and Tensor, a KV cache object with k_cache(i) /
// v_cache(i) / max_length() and a config struct. They bind here unchanged.
namespace backend_shape {
struct Config {
  int num_attention_heads, num_key_value_heads, head_dim;
  float rms_norm_eps, rope_theta;
};
struct LayerCache {
  std::vector<Tensor> k, v;
  int max_len;
  Tensor& k_cache(int i) { return k[i]; }
  Tensor& v_cache(int i) { return v[i]; }
  int max_length() const { return max_len; }
};
struct Buffers {
  Tensor q, k, v, attn_out, scores, decode_scores, rope_freq;
};
struct Layer {
  Tensor* q_norm_weight;
  Tensor* k_norm_weight;
};

// One layer's attention for seq_len tokens at start_pos, written as the
// backend writes it.
void attention_layer(Context& ctx, const Config& cfg_, LayerCache& kv_cache_, Buffers& buf_, Layer& layer, int i,
                     int seq_len, int start_pos) {
  if (seq_len == 1) {
    ops::decode_prepare_qkv(ctx, buf_.q, buf_.k, buf_.v, buf_.rope_freq, *layer.q_norm_weight, *layer.k_norm_weight,
                            kv_cache_.k_cache(i), kv_cache_.v_cache(i), start_pos, cfg_.num_attention_heads,
                            cfg_.num_key_value_heads, cfg_.head_dim, cfg_.rms_norm_eps, cfg_.rope_theta);
    ops::attention_decode(ctx, buf_.q, kv_cache_.k_cache(i), kv_cache_.v_cache(i), buf_.attn_out,
                          buf_.decode_scores, cfg_.num_attention_heads, cfg_.num_key_value_heads, cfg_.head_dim,
                          start_pos + 1);
    return;
  }
  ops::head_rms_norm(ctx, buf_.q, *layer.q_norm_weight, cfg_.rms_norm_eps, seq_len, cfg_.num_attention_heads,
                     cfg_.head_dim);
  ops::head_rms_norm(ctx, buf_.k, *layer.k_norm_weight, cfg_.rms_norm_eps, seq_len, cfg_.num_key_value_heads,
                     cfg_.head_dim);
  ops::apply_rope(ctx, buf_.q, buf_.k, seq_len, start_pos, cfg_.num_attention_heads, cfg_.num_key_value_heads,
                  cfg_.head_dim, cfg_.rope_theta);
  ops::copy_to_cache(ctx, buf_.k, kv_cache_.k_cache(i), seq_len, start_pos, cfg_.num_key_value_heads, cfg_.head_dim,
                     kv_cache_.max_length());
  ops::copy_to_cache(ctx, buf_.v, kv_cache_.v_cache(i), seq_len, start_pos, cfg_.num_key_value_heads, cfg_.head_dim,
                     kv_cache_.max_length());
  if (start_pos == 0)
    ops::attention_prefill(ctx, buf_.q, buf_.k, buf_.v, buf_.attn_out, buf_.scores, seq_len,
                           cfg_.num_attention_heads, cfg_.num_key_value_heads, cfg_.head_dim);
  else
    ops::attention_prefill_cached(ctx, buf_.q, kv_cache_.k_cache(i), kv_cache_.v_cache(i), buf_.attn_out,
                                  buf_.scores, seq_len, start_pos, cfg_.num_attention_heads,
                                  cfg_.num_key_value_heads, cfg_.head_dim, kv_cache_.max_length());
}
}  // namespace backend_shape

int main() {
  Context ctx;
  // ---- attention_decode with the reference backend's partials buffer ----
  {
    const int Hq = 16, Hkv = 4, D = 256, max_seq = 4096, L = 3001;
    const int max_tiles = (max_seq + 127) / 128;
    u16v q = rand_bf16(Hq * D), kc = rand_bf16(size_t(Hkv) * max_seq * D), vc = rand_bf16(size_t(Hkv) * max_seq * D);
    Tensor tq = upload(ctx, q, {1, Hq * D}, DType::bf16), tk = upload(ctx, kc, {Hkv, max_seq, D}, DType::bf16),
           tv = upload(ctx, vc, {Hkv, max_seq, D}, DType::bf16);
    Tensor out = Tensor::allocate(ctx, {1, Hq * D});
    Tensor scores = Tensor::allocate(ctx, {Hq, max_seq}, DType::f32);
    Tensor partials = Tensor::allocate(ctx, {Hq, max_tiles, 272}, DType::f32);
    u16v want(Hq * D);
    orc_attention_decode_baseline(q.data(), kc.data(), vc.data(), want.data(), 1, Hq, Hkv, D, max_seq, L);
    ops::attention_decode(ctx, tq, tk, tv, out, scores, Hq, Hkv, D, L, &partials);
    double e = relerr(download<uint16_t>(ctx, out), want);
    expect(e <= 1e-2, "attention_decode (split-K, backend partials)", e);
    ops::attention_decode(ctx, tq, tk, tv, out, scores, Hq, Hkv, D, L, nullptr);
    e = relerr(download<uint16_t>(ctx, out), want);
    expect(e <= 1e-2, "attention_decode (single pass)", e);
    // decode window with sinks (the AILA_ATTN_DECODE_* knobs as arguments)
    orc_attention_decode_window(q.data(), kc.data(), vc.data(), want.data(), 1, Hq, Hkv, D, max_seq, L, nullptr,
                                1000, -1, 6);
    ops::attention_decode_window(ctx, tq, tk, tv, out, scores, Hq, Hkv, D, L, &partials, 1000, -1, 6);
    e = relerr(download<uint16_t>(ctx, out), want);
    expect(e <= 1e-2, "attention_decode_window (window 1000, sink 6)", e);
  }
  // ---- prefill + copy_to_cache, fused variant, cached prefill -------------
  {
    const int S = 300, Hq = 32, Hkv = 8, D = 128, max_seq = 512, start = 100, S2 = 64;
    u16v q = rand_bf16(size_t(S) * Hq * D), k = rand_bf16(size_t(S) * Hkv * D), v = rand_bf16(size_t(S) * Hkv * D);
    Tensor tq = upload(ctx, q, {S, Hq * D}, DType::bf16), tk = upload(ctx, k, {S, Hkv * D}, DType::bf16),
           tv = upload(ctx, v, {S, Hkv * D}, DType::bf16);
    Tensor out = Tensor::allocate(ctx, {S, Hq * D}), scores = Tensor::allocate(ctx, {1}, DType::f32);
    Tensor kc = Tensor::allocate(ctx, {Hkv, max_seq, D}), vc = Tensor::allocate(ctx, {Hkv, max_seq, D});
    u16v want(size_t(S) * Hq * D);
    orc_attention_prefill_naive(q.data(), k.data(), v.data(), want.data(), S, Hq, Hkv, D);
    ops::copy_to_cache(ctx, tk, kc, S, start, Hkv, D, max_seq);
    ops::copy_to_cache(ctx, tv, vc, S, start, Hkv, D, max_seq);
    ops::attention_prefill(ctx, tq, tk, tv, out, scores, S, Hq, Hkv, D);
    double e = relerr(download<uint16_t>(ctx, out), want);
    expect(e <= 1e-2, "attention_prefill", e);
    u16v ck(size_t(Hkv) * max_seq * D, 0), cv(size_t(Hkv) * max_seq * D, 0);
    u16v got_k = download<uint16_t>(ctx, kc), got_v = download<uint16_t>(ctx, vc);
    orc_copy_to_cache(k.data(), ck.data(), S, start, Hkv, D, max_seq);
    orc_copy_to_cache(v.data(), cv.data(), S, start, Hkv, D, max_seq);
    bool same = true;
    for (int h = 0; h < Hkv; ++h)
      for (int r = start; r < start + S; ++r)
        same &= !std::memcmp(&got_k[(size_t(h) * max_seq + r) * D], &ck[(size_t(h) * max_seq + r) * D], D * 2) &&
                !std::memcmp(&got_v[(size_t(h) * max_seq + r) * D], &cv[(size_t(h) * max_seq + r) * D], D * 2);
    expect(same, "copy_to_cache (bit exact)", same ? 0 : 1);
    Tensor kc2 = Tensor::allocate(ctx, {Hkv, max_seq, D}), vc2 = Tensor::allocate(ctx, {Hkv, max_seq, D});
    ops::attention_prefill_write_cache(ctx, tq, tk, tv, out, kc2, vc2, S, start, Hq, Hkv, D, max_seq);
    e = relerr(download<uint16_t>(ctx, out), want);
    u16v got_k2 = download<uint16_t>(ctx, kc2);
    same = true;
    for (int h = 0; h < Hkv; ++h)
      same &= !std::memcmp(&got_k2[(size_t(h) * max_seq + start) * D], &ck[(size_t(h) * max_seq + start) * D],
                           size_t(S) * D * 2);
    expect(e <= 1e-2 && same, "attention_prefill_write_cache", e);
    // cached: S2 new queries at positions start+S .. attend the cache rows
    // [0, start+S+S2): fill rows [0,start) and [start+S, start+S+S2) too
    u16v full_k = rand_bf16(size_t(Hkv) * max_seq * D), full_v = rand_bf16(size_t(Hkv) * max_seq * D);
    Tensor fk = upload(ctx, full_k, {Hkv, max_seq, D}, DType::bf16), fv = upload(ctx, full_v, {Hkv, max_seq, D}, DType::bf16);
    u16v q2 = rand_bf16(size_t(S2) * Hq * D);
    Tensor tq2 = upload(ctx, q2, {S2, Hq * D}, DType::bf16), out2 = Tensor::allocate(ctx, {S2, Hq * D});
    ops::attention_prefill_cached(ctx, tq2, fk, fv, out2, scores, S2, start + S, Hq, Hkv, D, max_seq);
    u16v want2(size_t(S2) * Hq * D);
    orc_attention_prefill_cached(q2.data(), full_k.data(), full_v.data(), want2.data(), S2, start + S, Hq, Hkv, D,
                                 max_seq, 0);
    e = relerr(download<uint16_t>(ctx, out2), want2);
    expect(e <= 1e-2, "attention_prefill_cached", e);
  }
  // ---- attention_prefill_cached with the reference's score buffer: a short
  //      turn over a long prefix splits each query block's keys into runs ----
  {
    const int Hq = 16, Hkv = 4, D = 256, S = 100, start = 2100, max_seq = 2304;
    const int total = start + S;
    u16v kc = rand_bf16(size_t(Hkv) * max_seq * D), vc = rand_bf16(size_t(Hkv) * max_seq * D);
    u16v q = rand_bf16(size_t(S) * Hq * D);
    Tensor tk = upload(ctx, kc, {Hkv, max_seq, D}, DType::bf16), tv = upload(ctx, vc, {Hkv, max_seq, D}, DType::bf16);
    Tensor tq = upload(ctx, q, {S, Hq * D}, DType::bf16), out = Tensor::allocate(ctx, {S, Hq * D});
    Tensor scores = Tensor::allocate(ctx, {Hq, S, total}, DType::f32);   // as the backend sizes it
    // one run's records: {m, l, pad, acc[D]} fp32 per (head, row); the score
    // buffer holds total / (D + 4) runs, the split asks for up to 16
    const size_t need = aila_hip_gqa_prefill_cached_workspace_size(S, start, Hq, Hkv, D);
    const size_t per_run = size_t(Hq) * S * (D + 4) * sizeof(float);
    expect(need >= 2 * per_run && scores.size_bytes() >= 2 * per_run,
           "prefill_cached key split engages and scores_buf holds at least two runs", double(need / per_run));
    ops::attention_prefill_cached(ctx, tq, tk, tv, out, scores, S, start, Hq, Hkv, D, max_seq);
    u16v want(size_t(S) * Hq * D);
    orc_attention_prefill_cached(q.data(), kc.data(), vc.data(), want.data(), S, start, Hq, Hkv, D, max_seq, 0);
    const double e = relerr(download<uint16_t>(ctx, out), want);
    expect(e <= 1e-2, "attention_prefill_cached (key runs through scores_buf)", e);
    // unsupported head_dim must throw
    bool threw = false;
    try {
      ops::attention_prefill(ctx, tq, tk, tv, out, scores, S, Hq, Hkv, 96);
    } catch (const std::runtime_error&) {
      threw = true;
    }
    expect(threw, "attention_prefill rejects head_dim 96", 0);
  }
  // ---- DeltaNet: prefill then decode steps --------------------------------
  {
    const int T = 150, Hk = 2, Hv = 4, d = 128, steps = 3, total = T + steps;
    const float eps = 1e-6f, scale = 1.0f / std::sqrt(float(d));
    u16v q = rand_bf16(size_t(total) * Hk * d), k = rand_bf16(size_t(total) * Hk * d),
         v = rand_bf16(size_t(total) * Hv * d), a = rand_bf16(size_t(total) * Hv), b = rand_bf16(size_t(total) * Hv);
    std::vector<float> S0(size_t(Hv) * d * d);
    for (auto& x : S0) x = 0.02f * nrand();
    Tensor tq = upload(ctx, q, {total, Hk * d}, DType::bf16), tk = upload(ctx, k, {total, Hk * d}, DType::bf16),
           tv = upload(ctx, v, {total, Hv * d}, DType::bf16), ta = upload(ctx, a, {total, Hv}, DType::bf16),
           tb = upload(ctx, b, {total, Hv}, DType::bf16);
    Tensor st = upload(ctx, S0, {1, Hv, d, d}, DType::f32);
    Tensor out = Tensor::allocate(ctx, {total, Hv * d});
    Tensor ws = Tensor::allocate(ctx, {int64_t(ops::linear_delta_prefill_workspace_bytes(T, Hv, d, d))}, DType::u8);
    ops::linear_delta_prefill(ctx, tq, tk, tv, ta, tb, nullptr, nullptr, st, out, ws, T, Hk, Hv, d, d, eps, scale);
    for (int s = T; s < total; ++s) {
      Tensor vq = Tensor::view(ctx, tq.data_as<uint16_t>() + size_t(s) * Hk * d, {Hk * d});
      Tensor vk = Tensor::view(ctx, tk.data_as<uint16_t>() + size_t(s) * Hk * d, {Hk * d});
      Tensor vv = Tensor::view(ctx, tv.data_as<uint16_t>() + size_t(s) * Hv * d, {Hv * d});
      Tensor va = Tensor::view(ctx, ta.data_as<uint16_t>() + size_t(s) * Hv, {Hv});
      Tensor vb = Tensor::view(ctx, tb.data_as<uint16_t>() + size_t(s) * Hv, {Hv});
      Tensor vo = Tensor::view(ctx, out.data_as<uint16_t>() + size_t(s) * Hv * d, {Hv * d});
      ops::linear_delta_decode(ctx, vq, vk, vv, va, vb, nullptr, nullptr, st, vo, Hk, Hv, d, d, eps, scale);
    }
    std::vector<float> Sw = S0, of(size_t(total) * Hv * d);
    u16v ob(size_t(total) * Hv * d);
    orc_deltanet_recurrent(q.data(), k.data(), v.data(), a.data(), b.data(), nullptr, nullptr, Sw.data(), of.data(),
                           ob.data(), 1, total, Hk, Hv, d, d, eps, scale, 1);
    double es = relerr_f(download<float>(ctx, st), Sw);
    double eo = relerr(download<uint16_t>(ctx, out), ob);
    expect(es <= 1e-3, "linear_delta prefill+decode state", es);
    expect(eo <= 1e-2, "linear_delta prefill+decode outputs", eo);
  }
  // ---- QK-norm / RoPE / decode prep / output gate -------------------------
  {
    const int Hq = 16, Hkv = 4, D = 256, rot = 64, max_seq = 2048, pos = 1500, S = 40;
    const float eps = 1e-6f, theta = 1e7f;
    u16v qg = rand_bf16(size_t(Hq) * 2 * D), k = rand_bf16(size_t(Hkv) * D), v = rand_bf16(size_t(Hkv) * D);
    u16v qw = rand_bf16(D), kw = rand_bf16(D);
    Tensor tqg = upload(ctx, qg, {1, Hq * 2 * D}, DType::bf16), tk = upload(ctx, k, {1, Hkv * D}, DType::bf16),
           tv = upload(ctx, v, {1, Hkv * D}, DType::bf16), tqw = upload(ctx, qw, {D}, DType::bf16),
           tkw = upload(ctx, kw, {D}, DType::bf16);
    Tensor qo = Tensor::allocate(ctx, {1, Hq * D}), go = Tensor::allocate(ctx, {1, Hq * D});
    Tensor kc = Tensor::allocate(ctx, {Hkv, max_seq, D}), vc = Tensor::allocate(ctx, {Hkv, max_seq, D});
    ops::decode_prepare_qgkv_packed_partial(ctx, tqg, tk, tv, qo, go, tqw, tkw, kc, vc, pos, Hq, Hkv, D, eps, rot,
                                            theta);
    u16v wq(size_t(Hq) * D), wg(size_t(Hq) * D), wk = k;
    const int p1 = pos;
    orc_decode_prepare(qg.data(), 1, wq.data(), wg.data(), wk.data(), v.data(), qw.data(), kw.data(), nullptr,
                       nullptr, 1, Hq, Hkv, D, 0, rot, theta, eps, &p1);
    u16v gk = download<uint16_t>(ctx, tk), ck = download<uint16_t>(ctx, kc), cv = download<uint16_t>(ctx, vc);
    bool rows = true;
    for (int h = 0; h < Hkv; ++h)
      rows &= !std::memcmp(&ck[(size_t(h) * max_seq + pos) * D], &gk[size_t(h) * D], D * 2) &&
              !std::memcmp(&cv[(size_t(h) * max_seq + pos) * D], &v[size_t(h) * D], D * 2);
    double e = std::fmax(relerr(download<uint16_t>(ctx, qo), wq), relerr(gk, wk));
    expect(e <= 1e-2 && download<uint16_t>(ctx, go) == wg && rows, "decode_prepare_qgkv_packed_partial", e);
    // full rotary, q in place
    u16v q1 = rand_bf16(size_t(Hq) * D), k1 = rand_bf16(size_t(Hkv) * D);
    Tensor tq1 = upload(ctx, q1, {1, Hq * D}, DType::bf16), tk1 = upload(ctx, k1, {1, Hkv * D}, DType::bf16);
    Tensor freq = rope_freq_table(ctx, D, theta);
    ops::decode_prepare_qkv(ctx, tq1, tk1, tv, freq, tqw, tkw, kc, vc, 7, Hq, Hkv, D, eps, theta);
    u16v wq1(size_t(Hq) * D), wk1 = k1;
    const int p7 = 7;
    orc_decode_prepare(q1.data(), 0, wq1.data(), nullptr, wk1.data(), v.data(), qw.data(), kw.data(), nullptr,
                       nullptr, 1, Hq, Hkv, D, 0, D, theta, eps, &p7);
    e = std::fmax(relerr(download<uint16_t>(ctx, tq1), wq1), relerr(download<uint16_t>(ctx, tk1), wk1));
    expect(e <= 1e-2, "decode_prepare_qkv", e);
    // a rope_freq table that is not theta's: used as given
    {
      std::vector<float> tab(D / 2);
      for (int d = 0; d < D / 2; ++d) tab[d] = (d % 3 == 0 ? 0.5f : 1.0f) / std::pow(theta, (2.0f * d) / float(D));
      Tensor tfreq = upload(ctx, tab, {D / 2}, DType::f32);
      u16v q2 = rand_bf16(size_t(Hq) * D), k2 = rand_bf16(size_t(Hkv) * D);
      Tensor tq2 = upload(ctx, q2, {1, Hq * D}, DType::bf16), tk2 = upload(ctx, k2, {1, Hkv * D}, DType::bf16);
      ops::decode_prepare_qkv(ctx, tq2, tk2, tv, tfreq, tqw, tkw, kc, vc, 9, Hq, Hkv, D, eps, theta);
      orc_decode_prepare_qkv_freq(q2.data(), k2.data(), v.data(), tab.data(), qw.data(), kw.data(), nullptr, nullptr,
                                  9, Hq, Hkv, D, eps, 0);
      e = std::fmax(relerr(download<uint16_t>(ctx, tq2), q2), relerr(download<uint16_t>(ctx, tk2), k2));
      expect(e <= 1e-2, "decode_prepare_qkv (rope_freq table used as given)", e);
    }
    // prefill: head_rms_norm then apply_rope_partial with a text shift
    u16v xq = rand_bf16(size_t(S) * Hq * D), xk = rand_bf16(size_t(S) * Hkv * D);
    Tensor txq = upload(ctx, xq, {S, Hq * D}, DType::bf16), txk = upload(ctx, xk, {S, Hkv * D}, DType::bf16);
    ops::head_rms_norm(ctx, txq, tqw, eps, S, Hq, D);
    ops::head_rms_norm(ctx, txk, tkw, eps, S, Hkv, D);
    const int start = 10, prompt = 25, delta = -3;
    ops::apply_rope_partial(ctx, txq, txk, S, start, Hq, Hkv, D, rot, theta, false, nullptr, nullptr, nullptr,
                            prompt, delta);
    orc_head_rms_norm(xq.data(), qw.data(), nullptr, eps, S, Hq, D);
    orc_head_rms_norm(xk.data(), kw.data(), nullptr, eps, S, Hkv, D);
    const int n0 = prompt - start;
    orc_apply_rope(xq.data(), xk.data(), n0, start, Hq, Hkv, D, rot, theta);
    orc_apply_rope(xq.data() + size_t(n0) * Hq * D, xk.data() + size_t(n0) * Hkv * D, S - n0, prompt + delta, Hq,
                   Hkv, D, rot, theta);
    e = std::fmax(relerr(download<uint16_t>(ctx, txq), xq), relerr(download<uint16_t>(ctx, txk), xk));
    expect(e <= 1e-2, "head_rms_norm + apply_rope_partial (text shift)", e);
    // output gate, in place
    const int n = 100003;
    u16v a = rand_bf16(n), g = rand_bf16(n), wa(n);
    Tensor ta = upload(ctx, a, {n}, DType::bf16), tg = upload(ctx, g, {n}, DType::bf16);
    ops::sigmoid_mul(ctx, ta, tg, ta, n);
    orc_sigmoid_mul(a.data(), g.data(), wa.data(), n);
    e = relerr(download<uint16_t>(ctx, ta), wa);
    expect(e <= 1e-2, "sigmoid_mul", e);
    // interleaved mRoPE (prompt rows take their t/h/w streams, later rows
    // the shifted text position), prefill and decode forms
    {
      const int P = 30, dshift = -12, sec_t = 11, sec_h = 11, sec_w = 10;
      std::vector<int> pt(P), ph(P), pw(P);
      for (int i = 0; i < P; ++i) pt[i] = i / 3, ph[i] = (i * 7) % 11, pw[i] = (i * 5) % 13;
      Tensor tpt = upload(ctx, pt, {P}, DType::s32), tph = upload(ctx, ph, {P}, DType::s32),
             tpw = upload(ctx, pw, {P}, DType::s32);
      u16v mq = rand_bf16(size_t(S) * Hq * D), mk = rand_bf16(size_t(S) * Hkv * D);
      Tensor tmq = upload(ctx, mq, {S, Hq * D}, DType::bf16), tmk = upload(ctx, mk, {S, Hkv * D}, DType::bf16);
      ops::apply_rope_partial(ctx, tmq, tmk, S, start, Hq, Hkv, D, rot, theta, true, tpt.data_as<int>(),
                              tph.data_as<int>(), tpw.data_as<int>(), P, dshift, sec_t, sec_h, sec_w);
      orc_apply_rope_partial(mq.data(), mk.data(), S, start, Hq, Hkv, D, rot, theta, 1, pt.data(), ph.data(),
                             pw.data(), P, dshift, sec_t, sec_h, sec_w);
      e = std::fmax(relerr(download<uint16_t>(ctx, tmq), mq), relerr(download<uint16_t>(ctx, tmk), mk));
      expect(e <= 1e-2, "apply_rope_partial (interleaved mRoPE + text shift)", e);
      // decode step inside the prompt (streams) and past it (shift); cache row = start_pos
      for (const int sp : {P - 4, P + 40}) {
        u16v dq = rand_bf16(size_t(Hq) * 2 * D), dk = rand_bf16(size_t(Hkv) * D);
        Tensor tdq = upload(ctx, dq, {1, Hq * 2 * D}, DType::bf16), tdk = upload(ctx, dk, {1, Hkv * D}, DType::bf16);
        Tensor qo2 = Tensor::allocate(ctx, {1, Hq * D}), go2 = Tensor::allocate(ctx, {1, Hq * D});
        ops::decode_prepare_qgkv_packed_partial(ctx, tdq, tdk, tv, qo2, go2, tqw, tkw, kc, vc, sp, Hq, Hkv, D, eps,
                                                rot, theta, true, tpt.data_as<int>(), tph.data_as<int>(),
                                                tpw.data_as<int>(), P, dshift, sec_t, sec_h, sec_w);
        u16v wq2(size_t(Hq) * D), wg2(size_t(Hq) * D), wk2 = dk;
        orc_decode_prepare_rp(dq.data(), 1, wq2.data(), wg2.data(), wk2.data(), v.data(), qw.data(), kw.data(),
                              nullptr, nullptr, 1, Hq, Hkv, D, 0, rot, theta, eps, &sp, 1, pt.data(), ph.data(),
                              pw.data(), 0, P, dshift, nullptr, nullptr, sec_t, sec_h, sec_w);
        u16v gk2 = download<uint16_t>(ctx, tdk), ck2 = download<uint16_t>(ctx, kc);
        bool row_ok = true;
        for (int h = 0; h < Hkv; ++h)
          row_ok &= !std::memcmp(&ck2[(size_t(h) * max_seq + sp) * D], &gk2[size_t(h) * D], D * 2);
        e = std::fmax(relerr(download<uint16_t>(ctx, qo2), wq2), relerr(gk2, wk2));
        expect(e <= 1e-2 && row_ok && download<uint16_t>(ctx, go2) == wg2,
               sp < P ? "decode_prepare_qgkv_packed_partial (mRoPE, in prompt)"
                      : "decode_prepare_qgkv_packed_partial (text shift, cache row unshifted)",
               e);
      }
    }
  }
  // ---- whole DeltaNet layer: prefill over fused rows, then decode steps ----
  {
    const int Hk = 2, Hv = 4, d = 128, K = 4, T0 = 100, steps = 3, T = T0 + steps;
    const int ch = 2 * Hk * d + Hv * d, zd = Hv * d, all = ch + zd + 2 * Hv;
    const float eps = 1e-6f;
    u16v fused = rand_bf16(size_t(T) * all), w = rand_bf16(size_t(ch) * K), dtb = rand_bf16(Hv);
    std::vector<float> alog(Hv), nw(d), cs0(size_t(K - 1) * ch), S0(size_t(Hv) * d * d);
    for (auto& x : alog) x = 0.5f * nrand();
    for (auto& x : nw) x = 1.0f + 0.1f * nrand();
    for (auto& x : cs0) x = nrand();
    for (auto& x : S0) x = 0.02f * nrand();
    Tensor tf = upload(ctx, fused, {T, all}, DType::bf16), tw = upload(ctx, w, {ch, K}, DType::bf16),
           tdt = upload(ctx, dtb, {Hv}, DType::bf16), tal = upload(ctx, alog, {Hv}, DType::f32),
           tnw = upload(ctx, nw, {d}, DType::f32), tcs = upload(ctx, cs0, {K - 1, ch}, DType::f32),
           tst = upload(ctx, S0, {Hv, d, d}, DType::f32);
    Tensor out = Tensor::allocate(ctx, {T, zd});
    Tensor ws = Tensor::allocate(ctx, {int64_t(ops::linear_delta_layer_prefill_workspace_bytes(T0, Hk, Hv, d, d))},
                                 DType::u8);
    int head = 1;
    Tensor pre = Tensor::view(ctx, tf.data(), {T0, all});
    ops::linear_delta_layer_prefill(ctx, pre, out, T0, tw, tcs, head, &tdt, &tal, tnw, tst, ws, Hk, Hv, d, d, K, eps);
    for (int t = T0; t < T; ++t) {
      uint16_t* row = tf.data_as<uint16_t>() + size_t(t) * all;
      Tensor vq = Tensor::view(ctx, row, {1, ch}), vz = Tensor::view(ctx, row + ch, {1, zd}),
             va = Tensor::view(ctx, row + ch + zd, {1, Hv}), vb = Tensor::view(ctx, row + ch + zd + Hv, {1, Hv}),
             vo = Tensor::view(ctx, out.data_as<uint16_t>() + size_t(t) * zd, {1, zd});
      ops::linear_delta_layer_decode(ctx, vq, vz, va, vb, tw, tcs, head, &tdt, &tal, tnw, tst, vo, Hk, Hv, d, d, K,
                                     eps);
    }
    std::vector<float> Sw = S0, csw = cs0;
    u16v ow(size_t(T) * zd);
    orc_deltanet_layer(fused.data(), all, fused.data() + ch, all, fused.data() + ch + zd,
                       fused.data() + ch + zd + Hv, all, w.data(), csw.data(), 1, dtb.data(), alog.data(), nw.data(),
                       Sw.data(), ow.data(), 1, T, Hk, Hv, d, d, K, eps, 1.0f / std::sqrt(float(d)));
    const double es = relerr_f(download<float>(ctx, tst), Sw);
    const double eo = relerr(download<uint16_t>(ctx, out), ow);
    expect(es <= 1e-3 && eo <= 1e-2 && download<float>(ctx, tcs) == csw && head == (1 + T) % 3,
           "linear_delta_layer prefill + decode", std::fmax(es, eo));
  }
  // ---- attention_decode_paged: a shuffled page pool against the oracle -----
  {
    const int B = 2, Hq = 16, Hkv = 4, D = 256, page = 64, mp = 16, max_seq = page * mp;
    const int lens[B] = {700, 1024};
    const int npages = B * mp;
    u16v q = rand_bf16(size_t(B) * Hq * D);
    std::vector<u16v> kc(B), vc(B);
    u16v pk(size_t(npages) * Hkv * page * D), pv(pk.size());
    std::vector<int> table(size_t(B) * mp);
    for (int b = 0; b < B; ++b) {
      kc[b] = rand_bf16(size_t(Hkv) * max_seq * D);
      vc[b] = rand_bf16(size_t(Hkv) * max_seq * D);
      for (int j = 0; j < mp; ++j) {
        const int pg = ((b * mp + j) * 5) % npages;   // a permutation of the pool (gcd(5, 32) = 1)
        table[size_t(b) * mp + j] = pg;
        for (int h = 0; h < Hkv; ++h)
          std::memcpy(&pk[((size_t(pg) * Hkv + h) * page) * D], &kc[b][(size_t(h) * max_seq + j * page) * D],
                      size_t(page) * D * 2),
          std::memcpy(&pv[((size_t(pg) * Hkv + h) * page) * D], &vc[b][(size_t(h) * max_seq + j * page) * D],
                      size_t(page) * D * 2);
      }
    }
    Tensor tq = upload(ctx, q, {B, Hq * D}, DType::bf16);
    Tensor tpk = upload(ctx, pk, {npages, Hkv, page, D}, DType::bf16), tpv = upload(ctx, pv, {npages, Hkv, page, D}, DType::bf16);
    Tensor ttab = upload(ctx, table, {B, mp}, DType::s32);
    std::vector<int> lv(lens, lens + B);
    Tensor tlens = upload(ctx, lv, {B}, DType::s32);
    Tensor out = Tensor::allocate(ctx, {B, Hq * D});
    Tensor partials = Tensor::allocate(ctx, {B, Hq, mp, 16 + D}, DType::f32);
    ops::attention_decode_paged(ctx, tq, tpk, tpv, ttab, tlens, out, Hq, Hkv, D, max_seq, &partials);
    u16v got = download<uint16_t>(ctx, out);
    double e = 0;
    for (int b = 0; b < B; ++b) {
      u16v want(size_t(Hq) * D), gb(got.begin() + size_t(b) * Hq * D, got.begin() + size_t(b + 1) * Hq * D);
      orc_attention_decode_baseline(&q[size_t(b) * Hq * D], kc[b].data(), vc[b].data(), want.data(), 1, Hq, Hkv, D,
                                    max_seq, lens[b]);
      e = std::fmax(e, relerr(gb, want));
    }
    expect(e <= 1e-2, "attention_decode_paged (shuffled pool)", e);
  }
  // ---- the backend-shaped caller: prefill 40 tokens, then decode one ------
  {
    using namespace backend_shape;
    const Config cfg{16, 8, 128, 1e-6f, 1e6f};
    const int Hq = 16, Hkv = 8, D = 128, max_seq = 96, S = 40;
    LayerCache kv;
    kv.max_len = max_seq;
    kv.k.push_back(Tensor::allocate(ctx, {Hkv, max_seq, D}));
    kv.v.push_back(Tensor::allocate(ctx, {Hkv, max_seq, D}));
    u16v qw = rand_bf16(D), kw = rand_bf16(D);
    Tensor tqw = upload(ctx, qw, {D}, DType::bf16), tkw = upload(ctx, kw, {D}, DType::bf16);
    Layer layer{&tqw, &tkw};
    u16v q = rand_bf16(size_t(S) * Hq * D), k = rand_bf16(size_t(S) * Hkv * D), v = rand_bf16(size_t(S) * Hkv * D);
    Buffers buf;
    buf.q = upload(ctx, q, {S, Hq * D}, DType::bf16);
    buf.k = upload(ctx, k, {S, Hkv * D}, DType::bf16);
    buf.v = upload(ctx, v, {S, Hkv * D}, DType::bf16);
    buf.attn_out = Tensor::allocate(ctx, {S, Hq * D});
    buf.scores = Tensor::allocate(ctx, {1}, DType::f32);
    buf.decode_scores = Tensor::allocate(ctx, {Hq, max_seq}, DType::f32);
    buf.rope_freq = rope_freq_table(ctx, D, cfg.rope_theta);
    attention_layer(ctx, cfg, kv, buf, layer, 0, S, 0);
    u16v got_pre = download<uint16_t>(ctx, buf.attn_out);
    // oracle: norms, rope, cache, naive prefill
    u16v wq = q, wk = k, ck(size_t(Hkv) * max_seq * D, 0), cv(size_t(Hkv) * max_seq * D, 0), want(size_t(S) * Hq * D);
    orc_head_rms_norm(wq.data(), qw.data(), nullptr, cfg.rms_norm_eps, S, Hq, D);
    orc_head_rms_norm(wk.data(), kw.data(), nullptr, cfg.rms_norm_eps, S, Hkv, D);
    orc_apply_rope(wq.data(), wk.data(), S, 0, Hq, Hkv, D, D, cfg.rope_theta);
    orc_copy_to_cache(wk.data(), ck.data(), S, 0, Hkv, D, max_seq);
    orc_copy_to_cache(v.data(), cv.data(), S, 0, Hkv, D, max_seq);
    orc_attention_prefill_naive(wq.data(), wk.data(), v.data(), want.data(), S, Hq, Hkv, D);
    const double e1 = relerr(got_pre, want);
    // decode token S through the same statements
    u16v q1 = rand_bf16(size_t(Hq) * D), k1 = rand_bf16(size_t(Hkv) * D), v1 = rand_bf16(size_t(Hkv) * D);
    buf.q = upload(ctx, q1, {1, Hq * D}, DType::bf16);
    buf.k = upload(ctx, k1, {1, Hkv * D}, DType::bf16);
    buf.v = upload(ctx, v1, {1, Hkv * D}, DType::bf16);
    buf.attn_out = Tensor::allocate(ctx, {1, Hq * D});
    attention_layer(ctx, cfg, kv, buf, layer, 0, 1, S);
    u16v got_dec = download<uint16_t>(ctx, buf.attn_out);
    u16v want_dec(size_t(Hq) * D);
    orc_decode_prepare_qkv(q1.data(), k1.data(), v1.data(), qw.data(), kw.data(), ck.data(), cv.data(), S, Hq, Hkv,
                           D, cfg.rms_norm_eps, cfg.rope_theta, max_seq);
    orc_attention_decode_baseline(q1.data(), ck.data(), cv.data(), want_dec.data(), 1, Hq, Hkv, D, max_seq, S + 1);
    const double e2 = relerr(got_dec, want_dec);
    u16v gk = download<uint16_t>(ctx, kv.k_cache(0)), gv = download<uint16_t>(ctx, kv.v_cache(0));
    // rows [0, S] of every head (rows past them were never written); the
    // k rows went through the GPU's norm and rotation, so to tolerance
    u16v rk, rv, wrk, wrv;
    for (int h = 0; h < Hkv; ++h) {
      const size_t o = size_t(h) * max_seq * D, n = size_t(S + 1) * D;
      rk.insert(rk.end(), gk.begin() + o, gk.begin() + o + n);
      wrk.insert(wrk.end(), ck.begin() + o, ck.begin() + o + n);
      rv.insert(rv.end(), gv.begin() + o, gv.begin() + o + n);
      wrv.insert(wrv.end(), cv.begin() + o, cv.begin() + o + n);
    }
    const bool cache_ok = relerr(rk, wrk) <= 1e-2 && rv == wrv;
    expect(e1 <= 1e-2 && e2 <= 1e-2 && cache_ok, "backend-shaped ops:: caller (prefill, decode)", std::fmax(e1, e2));
  }
  std::printf("peak device bytes %zu\n", ctx.peak_allocated_bytes());
  std::printf(g_fail ? "FAILED %d\n" : "ALL OK\n", g_fail);
  return g_fail ? 1 : 0;
}

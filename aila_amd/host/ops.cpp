// ops:: over the C ABI (see Ops.hpp).
#include "Ops.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <stdexcept>
#include <string>

#include "aila_hip.h"

namespace ops {
namespace {

void check(int rc, const char* what) {
  if (rc != AILA_HIP_OK)
    throw std::runtime_error(std::string(what) + ": " + aila_hip_last_error());
}

void need_dtype(const Tensor& t, DType dt, const char* name) {
  if (!t.valid()) throw std::runtime_error(std::string(name) + ": invalid tensor");
  if (t.dtype() != dt) throw std::runtime_error(std::string(name) + ": wrong dtype");
}

}  // namespace

void copy_to_cache(Context& ctx, Tensor& new_kv, Tensor& cache, int seq_len, int start_pos,
                   int num_heads, int head_dim, int max_seq_len) {
  need_dtype(new_kv, DType::bf16, "copy_to_cache new_kv");
  need_dtype(cache, DType::bf16, "copy_to_cache cache");
  check(aila_hip_copy_to_cache(new_kv.data(), cache.data(), seq_len, start_pos, num_heads, head_dim,
                               max_seq_len, ctx.stream()),
        "copy_to_cache");
}

namespace {
int env_int(const char* name, int dflt) {
  const char* v = std::getenv(name);
  if (v == nullptr || *v == '\0') return dflt;
  char* end = nullptr;
  const long x = std::strtol(v, &end, 10);
  return end && *end == '\0' ? static_cast<int>(x) : dflt;
}
}  // namespace

void attention_decode(Context& ctx, Tensor& q, Tensor& k_cache, Tensor& v_cache, Tensor& output,
                      Tensor& scores_buf, int num_heads, int num_kv_heads, int head_dim,
                      int cached_len, Tensor* exact_partials_buf) {
  // The reference's decode window knobs, read once (AttentionOps.cpp:517-551).
  static const int window = std::max(0, env_int("AILA_ATTN_DECODE_WINDOW", 0));
  static const int window_start = env_int("AILA_ATTN_DECODE_WINDOW_START", -1);
  static const int sink = std::max(0, env_int("AILA_ATTN_DECODE_SINK", 0));
  attention_decode_window(ctx, q, k_cache, v_cache, output, scores_buf, num_heads, num_kv_heads, head_dim,
                          cached_len, exact_partials_buf, window, window_start, sink);
}

void attention_decode_window(Context& ctx, Tensor& q, Tensor& k_cache, Tensor& v_cache, Tensor& output,
                             Tensor& scores_buf, int num_heads, int num_kv_heads, int head_dim, int cached_len,
                             Tensor* exact_partials_buf, int window, int window_start, int sink) {
  (void)scores_buf;
  need_dtype(q, DType::bf16, "attention_decode q");
  need_dtype(k_cache, DType::bf16, "attention_decode k_cache");
  need_dtype(v_cache, DType::bf16, "attention_decode v_cache");
  need_dtype(output, DType::bf16, "attention_decode output");
  const int max_seq = static_cast<int>(k_cache.shape(1));
  void* ws = nullptr;
  size_t ws_bytes = 0;
  if (exact_partials_buf && exact_partials_buf->valid()) {
    ws = exact_partials_buf->data();
    ws_bytes = exact_partials_buf->size_bytes();
    // a buffer too small for two records per head falls back to one pass
    if (ws_bytes < 2 * static_cast<size_t>(num_heads) * (16 + head_dim) * sizeof(float)) {
      ws = nullptr;
      ws_bytes = 0;
    }
  }
  if (window > 0)
    check(aila_hip_gqa_decode_window(q.data(), k_cache.data(), v_cache.data(), output.data(), ws, ws_bytes, 1,
                                     num_heads, num_kv_heads, head_dim, max_seq, cached_len, nullptr, window,
                                     window_start, sink, ctx.stream()),
          "attention_decode");
  else
    check(aila_hip_gqa_decode(q.data(), k_cache.data(), v_cache.data(), output.data(), ws, ws_bytes, 1,
                              num_heads, num_kv_heads, head_dim, max_seq, cached_len, nullptr,
                              ctx.stream()),
          "attention_decode");
}

void attention_decode_paged(Context& ctx, Tensor& q, Tensor& k_pages, Tensor& v_pages, Tensor& block_table,
                            Tensor& seq_lens, Tensor& output, int num_heads, int num_kv_heads, int head_dim,
                            int max_len, Tensor* exact_partials_buf) {
  need_dtype(q, DType::bf16, "attention_decode_paged q");
  need_dtype(k_pages, DType::bf16, "attention_decode_paged k_pages");
  need_dtype(v_pages, DType::bf16, "attention_decode_paged v_pages");
  need_dtype(output, DType::bf16, "attention_decode_paged output");
  need_dtype(block_table, DType::s32, "attention_decode_paged block_table");
  need_dtype(seq_lens, DType::s32, "attention_decode_paged seq_lens");
  const int B = static_cast<int>(block_table.shape(0));
  const int max_pages = static_cast<int>(block_table.shape(1));
  const int page_size = static_cast<int>(k_pages.shape(2));
  void* ws = nullptr;
  size_t ws_bytes = 0;
  if (exact_partials_buf && exact_partials_buf->valid() &&
      exact_partials_buf->size_bytes() >= 2 * static_cast<size_t>(B) * num_heads * (16 + head_dim) * sizeof(float)) {
    ws = exact_partials_buf->data();
    ws_bytes = exact_partials_buf->size_bytes();
  }
  check(aila_hip_gqa_decode_paged(q.data(), k_pages.data(), v_pages.data(), output.data(), ws, ws_bytes, B,
                                  num_heads, num_kv_heads, head_dim, page_size,
                                  static_cast<const int*>(block_table.data()), max_pages, max_len,
                                  static_cast<const int*>(seq_lens.data()), ctx.stream()),
        "attention_decode_paged");
}

void attention_prefill(Context& ctx, Tensor& q, Tensor& k, Tensor& v, Tensor& output,
                       Tensor& scores_buf, int seq_len, int num_heads, int num_kv_heads,
                       int head_dim) {
  (void)scores_buf;
  need_dtype(q, DType::bf16, "attention_prefill q");
  check(aila_hip_gqa_prefill(q.data(), k.data(), v.data(), output.data(), nullptr, nullptr, 0, 0, seq_len,
                             num_heads, num_kv_heads, head_dim, ctx.stream()),
        "attention_prefill");
}

void attention_prefill_write_cache(Context& ctx, Tensor& q, Tensor& k, Tensor& v, Tensor& output,
                                   Tensor& k_cache, Tensor& v_cache, int seq_len, int start_pos,
                                   int num_heads, int num_kv_heads, int head_dim, int max_seq_len) {
  need_dtype(q, DType::bf16, "attention_prefill_write_cache q");
  check(aila_hip_gqa_prefill(q.data(), k.data(), v.data(), output.data(), k_cache.data(), v_cache.data(),
                             start_pos, max_seq_len, seq_len, num_heads, num_kv_heads, head_dim,
                             ctx.stream()),
        "attention_prefill_write_cache");
}

void attention_prefill_cached(Context& ctx, Tensor& q, Tensor& k_cache, Tensor& v_cache,
                              Tensor& output, Tensor& scores_buf, int seq_len, int start_pos,
                              int num_heads, int num_kv_heads, int head_dim, int max_seq_len) {
  need_dtype(q, DType::bf16, "attention_prefill_cached q");
  // The reference's score buffer ([heads, seq, total] fp32, never
  // materialised here) serves as the key-split workspace.
  const bool ws = scores_buf.valid();
  check(aila_hip_gqa_prefill_cached_ws(q.data(), k_cache.data(), v_cache.data(), output.data(),
                                       ws ? scores_buf.data() : nullptr, ws ? scores_buf.size_bytes() : 0, seq_len,
                                       start_pos, num_heads, num_kv_heads, head_dim, max_seq_len, ctx.stream()),
        "attention_prefill_cached");
}

void linear_delta_decode(Context& ctx, Tensor& q, Tensor& k, Tensor& v, Tensor& a, Tensor& b,
                         Tensor* dt_bias, Tensor* A_log, Tensor& state, Tensor& out,
                         int num_k_heads, int num_v_heads, int head_k_dim, int head_v_dim,
                         float eps, float scale) {
  need_dtype(state, DType::f32, "linear_delta_decode state");
  const int B = state.ndim() == 4 ? static_cast<int>(state.shape(0)) : 1;
  check(aila_hip_deltanet_decode(q.data(), k.data(), v.data(), a.data(), b.data(),
                                 dt_bias ? dt_bias->data() : nullptr,
                                 A_log ? static_cast<const float*>(A_log->data()) : nullptr,
                                 static_cast<float*>(state.data()), out.data(), B, num_k_heads,
                                 num_v_heads, head_k_dim, head_v_dim, eps, scale, ctx.stream()),
        "linear_delta_decode");
}

size_t linear_delta_prefill_workspace_bytes(int seq_len, int num_v_heads, int head_k_dim,
                                            int head_v_dim) {
  return aila_hip_deltanet_prefill_workspace_size(1, seq_len, num_v_heads, head_k_dim, head_v_dim);
}

void linear_delta_prefill(Context& ctx, Tensor& q, Tensor& k, Tensor& v, Tensor& a, Tensor& b,
                          Tensor* dt_bias, Tensor* A_log, Tensor& state, Tensor& out,
                          Tensor& workspace, int seq_len, int num_k_heads, int num_v_heads,
                          int head_k_dim, int head_v_dim, float eps, float scale) {
  need_dtype(state, DType::f32, "linear_delta_prefill state");
  check(aila_hip_deltanet_prefill(q.data(), k.data(), v.data(), a.data(), b.data(),
                                  dt_bias ? dt_bias->data() : nullptr,
                                  A_log ? static_cast<const float*>(A_log->data()) : nullptr,
                                  static_cast<float*>(state.data()), out.data(), workspace.data(),
                                  workspace.size_bytes(), 1, seq_len, num_k_heads, num_v_heads,
                                  head_k_dim, head_v_dim, eps, scale, ctx.stream()),
        "linear_delta_prefill");
}

namespace {

void* opt(Tensor& t) { return t.valid() ? t.data() : nullptr; }

// The reference's rotary position arguments (ElementwiseOps.cpp:33-103,
// 555-863) as the C ABI's position record. The position streams are the
// engine's device arrays, indexed by cache row.
aila_hip_rope_pos rope_pos(bool interleaved, const int* pos_t, const int* pos_h, const int* pos_w,
                           int prompt_pos_len, int text_pos_delta, int sec_t, int sec_h, int sec_w) {
  aila_hip_rope_pos rp{};
  rp.interleaved = interleaved ? 1 : 0;
  rp.pos_t = pos_t;
  rp.pos_h = pos_h;
  rp.pos_w = pos_w;
  rp.pos_stride = 0;
  rp.prompt_pos_len = prompt_pos_len;
  rp.text_pos_delta = text_pos_delta;
  rp.mrope_section_t = sec_t;
  rp.mrope_section_h = sec_h;
  rp.mrope_section_w = sec_w;
  return rp;
}

}  // namespace

void head_rms_norm(Context& ctx, Tensor& x, Tensor& weight, float eps, int seq_len, int num_heads,
                   int head_dim) {
  need_dtype(x, DType::bf16, "head_rms_norm x");
  if (weight.valid()) need_dtype(weight, DType::bf16, "head_rms_norm weight");
  check(aila_hip_head_rms_norm(x.data(), opt(weight), seq_len, num_heads, head_dim, eps, ctx.stream()),
        "head_rms_norm");
}

void sigmoid_mul(Context& ctx, Tensor& input, Tensor& gate, Tensor& output, int n) {
  need_dtype(input, DType::bf16, "sigmoid_mul input");
  need_dtype(gate, DType::bf16, "sigmoid_mul gate");
  need_dtype(output, DType::bf16, "sigmoid_mul output");
  check(aila_hip_sigmoid_mul(input.data(), gate.data(), output.data(), n, ctx.stream()), "sigmoid_mul");
}

void apply_rope(Context& ctx, Tensor& q, Tensor& k, int seq_len, int start_pos, int num_heads_q,
                int num_kv_heads, int head_dim, float theta) {
  apply_rope_partial(ctx, q, k, seq_len, start_pos, num_heads_q, num_kv_heads, head_dim, head_dim, theta);
}

void apply_rope_partial(Context& ctx, Tensor& q, Tensor& k, int seq_len, int start_pos, int num_heads_q,
                        int num_kv_heads, int head_dim, int rotary_dim, float theta, bool interleaved,
                        const int* pos_t, const int* pos_h, const int* pos_w, int prompt_pos_len,
                        int text_pos_delta, int mrope_section_t, int mrope_section_h, int mrope_section_w) {
  need_dtype(q, DType::bf16, "apply_rope q");
  need_dtype(k, DType::bf16, "apply_rope k");
  const aila_hip_rope_pos rp = rope_pos(interleaved, pos_t, pos_h, pos_w, prompt_pos_len, text_pos_delta,
                                        mrope_section_t, mrope_section_h, mrope_section_w);
  check(aila_hip_apply_rope(q.data(), k.data(), seq_len, start_pos, num_heads_q, num_kv_heads, head_dim, rotary_dim,
                            theta, &rp, ctx.stream()),
        "apply_rope_partial");
}

void decode_prepare_qkv(Context& ctx, Tensor& q, Tensor& k, Tensor& v, Tensor& rope_freq,
                        Tensor& q_norm_weight, Tensor& k_norm_weight, Tensor& k_cache, Tensor& v_cache,
                        int start_pos, int num_heads_q, int num_kv_heads, int head_dim, float eps,
                        float theta) {
  // angle = start_pos * rope_freq[d] (ElementwiseOps.cpp:159, 198): the
  // table is used as given (an invalid tensor falls back to theta)
  for (Tensor* t : {&q, &k, &v, &k_cache, &v_cache}) need_dtype(*t, DType::bf16, "decode_prepare_qkv");
  aila_hip_rope_pos rp{};
  if (rope_freq.valid()) {
    need_dtype(rope_freq, DType::f32, "decode_prepare_qkv rope_freq");
    if (rope_freq.numel() < head_dim / 2) throw std::runtime_error("decode_prepare_qkv: rope_freq holds < head_dim/2 values");
    rp.inv_freq = rope_freq.data_as<float>();
  }
  check(aila_hip_decode_prepare_qkv(q.data(), 0, q.data(), nullptr, k.data(), v.data(), opt(q_norm_weight),
                                    opt(k_norm_weight), k_cache.data(), v_cache.data(), 1, num_heads_q,
                                    num_kv_heads, head_dim, static_cast<int>(k_cache.shape(1)), head_dim, theta,
                                    eps, start_pos, nullptr, &rp, ctx.stream()),
        "decode_prepare_qkv");
}

void decode_prepare_qkv_partial(Context& ctx, Tensor& q, Tensor& k, Tensor& v, Tensor& q_norm_weight,
                                Tensor& k_norm_weight, Tensor& k_cache, Tensor& v_cache, int start_pos,
                                int num_heads_q, int num_kv_heads, int head_dim, float eps, int rotary_dim,
                                float theta, bool interleaved, const int* pos_t, const int* pos_h,
                                const int* pos_w, int prompt_pos_len, int text_pos_delta, int mrope_section_t,
                                int mrope_section_h, int mrope_section_w) {
  const aila_hip_rope_pos rp = rope_pos(interleaved, pos_t, pos_h, pos_w, prompt_pos_len, text_pos_delta,
                                        mrope_section_t, mrope_section_h, mrope_section_w);
  for (Tensor* t : {&q, &k, &v, &k_cache, &v_cache}) need_dtype(*t, DType::bf16, "decode_prepare_qkv");
  check(aila_hip_decode_prepare_qkv(q.data(), 0, q.data(), nullptr, k.data(), v.data(), opt(q_norm_weight),
                                    opt(k_norm_weight), k_cache.data(), v_cache.data(), 1, num_heads_q,
                                    num_kv_heads, head_dim, static_cast<int>(k_cache.shape(1)), rotary_dim,
                                    theta, eps, start_pos, nullptr, &rp, ctx.stream()),
        "decode_prepare_qkv");
}

void decode_prepare_qgkv_packed_partial(Context& ctx, Tensor& q_gate_packed, Tensor& k, Tensor& v,
                                        Tensor& q_out, Tensor& gate_out, Tensor& q_norm_weight,
                                        Tensor& k_norm_weight, Tensor& k_cache, Tensor& v_cache,
                                        int start_pos, int num_heads_q, int num_kv_heads, int head_dim,
                                        float eps, int rotary_dim, float theta, bool interleaved,
                                        const int* pos_t, const int* pos_h, const int* pos_w,
                                        int prompt_pos_len, int text_pos_delta, int mrope_section_t,
                                        int mrope_section_h, int mrope_section_w) {
  const aila_hip_rope_pos rp = rope_pos(interleaved, pos_t, pos_h, pos_w, prompt_pos_len, text_pos_delta,
                                        mrope_section_t, mrope_section_h, mrope_section_w);
  for (Tensor* t : {&q_gate_packed, &k, &v, &q_out, &gate_out, &k_cache, &v_cache})
    need_dtype(*t, DType::bf16, "decode_prepare_qgkv_packed_partial");
  check(aila_hip_decode_prepare_qkv(q_gate_packed.data(), 1, q_out.data(), gate_out.data(), k.data(), v.data(),
                                    opt(q_norm_weight), opt(k_norm_weight), k_cache.data(), v_cache.data(), 1,
                                    num_heads_q, num_kv_heads, head_dim, static_cast<int>(k_cache.shape(1)),
                                    rotary_dim, theta, eps, start_pos, nullptr, &rp, ctx.stream()),
        "decode_prepare_qgkv_packed_partial");
}

void linear_delta_layer_decode(Context& ctx, Tensor& qkv, Tensor& z, Tensor& a, Tensor& b, Tensor& conv1d_weight,
                               Tensor& conv_state, int& conv_head, Tensor* dt_bias, Tensor* A_log,
                               Tensor& norm_weight, Tensor& state, Tensor& out, int num_k_heads, int num_v_heads,
                               int head_k_dim, int head_v_dim, int conv_kernel, float eps, Tensor* arrivals) {
  for (Tensor* t : {&qkv, &z, &a, &b, &conv1d_weight, &out}) need_dtype(*t, DType::bf16, "linear_delta_layer_decode");
  if (arrivals) need_dtype(*arrivals, DType::s32, "linear_delta_layer_decode arrivals");
  for (Tensor* t : {&conv_state, &state, &norm_weight}) need_dtype(*t, DType::f32, "linear_delta_layer_decode");
  const int ch = 2 * num_k_heads * head_k_dim + num_v_heads * head_v_dim;
  const float scale = 1.0f / std::sqrt(static_cast<float>(head_k_dim));
  check(aila_hip_deltanet_layer_decode(qkv.data(), ch, z.data(), num_v_heads * head_v_dim, a.data(), b.data(),
                                       num_v_heads, conv1d_weight.data(), conv_state.data_as<float>(), conv_head,
                                       nullptr, dt_bias ? dt_bias->data() : nullptr,
                                       A_log ? A_log->data_as<float>() : nullptr, norm_weight.data_as<float>(),
                                       state.data_as<float>(), out.data(), 1, num_k_heads, num_v_heads, head_k_dim,
                                       head_v_dim, conv_kernel, eps, scale,
                                       arrivals ? static_cast<unsigned int*>(arrivals->data()) : nullptr, ctx.stream()),
        "linear_delta_layer_decode");
  if (conv_kernel > 1) conv_head = (conv_head + 1) % (conv_kernel - 1);
}

size_t linear_delta_layer_prefill_workspace_bytes(int seq_len, int num_k_heads, int num_v_heads, int head_k_dim,
                                                  int head_v_dim) {
  return aila_hip_deltanet_layer_prefill_workspace_size(1, seq_len, num_k_heads, num_v_heads, head_k_dim,
                                                        head_v_dim);
}

void linear_delta_layer_prefill(Context& ctx, Tensor& fused_all, Tensor& out, int seq_len, Tensor& conv1d_weight,
                                Tensor& conv_state, int& conv_head, Tensor* dt_bias, Tensor* A_log,
                                Tensor& norm_weight, Tensor& state, Tensor& workspace, int num_k_heads,
                                int num_v_heads, int head_k_dim, int head_v_dim, int conv_kernel, float eps) {
  for (Tensor* t : {&fused_all, &conv1d_weight, &out}) need_dtype(*t, DType::bf16, "linear_delta_layer_prefill");
  for (Tensor* t : {&conv_state, &state, &norm_weight}) need_dtype(*t, DType::f32, "linear_delta_layer_prefill");
  const int ch = 2 * num_k_heads * head_k_dim + num_v_heads * head_v_dim;
  const int zd = num_v_heads * head_v_dim;
  const int all_dim = ch + zd + 2 * num_v_heads;
  const float scale = 1.0f / std::sqrt(static_cast<float>(head_k_dim));
  uint16_t* row = fused_all.data_as<uint16_t>();
  check(aila_hip_deltanet_layer_prefill(row, all_dim, row + ch, all_dim, row + ch + zd, row + ch + zd + num_v_heads,
                                        all_dim, conv1d_weight.data(), conv_state.data_as<float>(), conv_head,
                                        dt_bias ? dt_bias->data() : nullptr, A_log ? A_log->data_as<float>() : nullptr,
                                        norm_weight.data_as<float>(), state.data_as<float>(), out.data(),
                                        workspace.data(), workspace.size_bytes(), 1, seq_len, num_k_heads,
                                        num_v_heads, head_k_dim, head_v_dim, conv_kernel, eps, scale, ctx.stream()),
        "linear_delta_layer_prefill");
  if (conv_kernel > 1) conv_head = (conv_head + seq_len) % (conv_kernel - 1);
}

}  // namespace ops

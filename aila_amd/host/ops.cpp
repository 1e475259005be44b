// ops:: over the C ABI (see Ops.hpp).
#include "Ops.hpp"

#include <stdexcept>
#include <string>

#include "aila_hip.h"

namespace aila {
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

void attention_decode(Context& ctx, Tensor& q, Tensor& k_cache, Tensor& v_cache, Tensor& output,
                      Tensor& scores_buf, int num_heads, int num_kv_heads, int head_dim,
                      int cached_len, Tensor* exact_partials_buf) {
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
  check(aila_hip_gqa_decode(q.data(), k_cache.data(), v_cache.data(), output.data(), ws, ws_bytes, 1,
                            num_heads, num_kv_heads, head_dim, max_seq, cached_len, nullptr,
                            ctx.stream()),
        "attention_decode");
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
  (void)scores_buf;
  need_dtype(q, DType::bf16, "attention_prefill_cached q");
  check(aila_hip_gqa_prefill_cached(q.data(), k_cache.data(), v_cache.data(), output.data(), seq_len,
                                    start_pos, num_heads, num_kv_heads, head_dim, max_seq_len,
                                    ctx.stream()),
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

}  // namespace ops
}  // namespace aila

// ops:: attention hot path on MI355X: the reference's operator interface
// (Aila src/ops/Ops.hpp:196-298) with the same names, argument order and
// meaning, implemented over the C ABI in include/aila_hip.h. Every op
// enqueues on ctx.stream() and returns before completion; failures of the
// underlying C ABI (bad shapes, unsupported head_dim, launch errors) are
// thrown as std::runtime_error.
#pragma once

#include "Context.hpp"
#include "Tensor.hpp"

// The reference declares these at top level (namespace ops, Ops.hpp:139)
// over global Context and Tensor classes (src/core/Context.hpp:14,
// Tensor.hpp:15); Context.hpp and Tensor.hpp here export aila::Context and
// aila::Tensor at global scope, so the backends' unqualified
// ops::attention_decode(ctx, ...) calls bind unchanged.
namespace ops {

// new_kv [seq_len, num_heads*head_dim] -> cache [num_heads, max_seq_len,
// head_dim] at start_pos (Ops.hpp:196-201).
void copy_to_cache(Context& ctx, Tensor& new_kv, Tensor& cache, int seq_len, int start_pos,
                   int num_heads, int head_dim, int max_seq_len);

// Single-token GQA decode (Ops.hpp:259-269). q [1, Hq*D]; k_cache/v_cache
// [Hkv, max_seq, D] (max_seq read from k_cache.shape(1), as the reference
// does at AttentionOps.cpp:87); output [1, Hq*D]. scores_buf is accepted and
// unused. exact_partials_buf (fp32, e.g. the backend's [Hq, max_tiles, 272]
// buffer) enables split-K with as many splits as it holds records; null runs
// the single-pass kernel. Like the reference it reads the decode window
// knobs AILA_ATTN_DECODE_WINDOW / _WINDOW_START / _SINK once
// (AttentionOps.cpp:517-551; window 0, the default, attends every row).
void attention_decode(Context& ctx, Tensor& q, Tensor& k_cache, Tensor& v_cache, Tensor& output,
                      Tensor& scores_buf, int num_heads, int num_kv_heads, int head_dim,
                      int cached_len, Tensor* exact_partials_buf = nullptr);

// The same with the window knobs as arguments: a sequence of more than
// window_start rows (< 0: max(512, window)) attends its first `sink` and last
// `window` rows only (AttentionOps.cpp:598-616).
void attention_decode_window(Context& ctx, Tensor& q, Tensor& k_cache, Tensor& v_cache, Tensor& output,
                             Tensor& scores_buf, int num_heads, int num_kv_heads, int head_dim, int cached_len,
                             Tensor* exact_partials_buf, int window, int window_start, int sink);

// The same decode over a paged KV cache (an addition behind the same shim;
// the reference keeps one contiguous cache per sequence): k_pages/v_pages
// [num_pages, Hkv, page_size, D] bf16, block_table s32 [B, max_pages] (row
// t of sequence b is row t % page_size of page block_table[b][t /
// page_size]), seq_lens s32 [B]; q/output [B, Hq*D]. max_len bounds every
// seq_lens[b]; page_size is a multiple of 16. exact_partials_buf as above.
void attention_decode_paged(Context& ctx, Tensor& q, Tensor& k_pages, Tensor& v_pages, Tensor& block_table,
                            Tensor& seq_lens, Tensor& output, int num_heads, int num_kv_heads, int head_dim,
                            int max_len, Tensor* exact_partials_buf = nullptr);

// Causal prefill over the current chunk (Ops.hpp:271-282). q [S, Hq*D],
// k/v [S, Hkv*D]; output [S, Hq*D]. scores_buf is accepted and unused (no
// [H, S, S] score matrix is materialised).
void attention_prefill(Context& ctx, Tensor& q, Tensor& k, Tensor& v, Tensor& output,
                       Tensor& scores_buf, int seq_len, int num_heads, int num_kv_heads,
                       int head_dim);

// attention_prefill fused with the two copy_to_cache calls that precede it in
// the backends (Qwen3DenseBackend.cpp:318-325): k/v are also written to the
// caches at start_pos. Addition; the reference issues three ops.
void attention_prefill_write_cache(Context& ctx, Tensor& q, Tensor& k, Tensor& v, Tensor& output,
                                   Tensor& k_cache, Tensor& v_cache, int seq_len, int start_pos,
                                   int num_heads, int num_kv_heads, int head_dim, int max_seq_len);

// Incremental prefill against the cache (Ops.hpp:284-298).
void attention_prefill_cached(Context& ctx, Tensor& q, Tensor& k_cache, Tensor& v_cache,
                              Tensor& output, Tensor& scores_buf, int seq_len, int start_pos,
                              int num_heads, int num_kv_heads, int head_dim, int max_seq_len);

// Gated DeltaNet recurrence, one token (the state update of
// Qwen35HybridTextBackend::run_linear_delta_decode_gpu,
// Qwen35HybridTextBackend.cpp:975-1166, after conv1d/SiLU and before the
// gated RMSNorm). q,k [Hk*dk] bf16, v [Hv*dv] bf16, a,b [Hv] bf16 (one
// sequence; batch via the leading dim of state [B, Hv, dk, dv] fp32),
// out [Hv*dv] bf16 = scale * S^T q. dt_bias (bf16 [Hv]) and A_log (fp32 [Hv])
// may be null.
void linear_delta_decode(Context& ctx, Tensor& q, Tensor& k, Tensor& v, Tensor& a, Tensor& b,
                         Tensor* dt_bias, Tensor* A_log, Tensor& state, Tensor& out,
                         int num_k_heads, int num_v_heads, int head_k_dim, int head_v_dim,
                         float eps, float scale);

// Chunked prefill of the same recurrence over seq_len tokens (replaces the
// token-sequential run_linear_delta_prefill_gpu_batched,
// Qwen35HybridTextBackend.cpp:1306-1508). q,k [S, Hk*dk]; v [S, Hv*dv];
// a,b [S, Hv]; out [S, Hv*dv]; workspace u8 of at least
// linear_delta_prefill_workspace_bytes(...).
size_t linear_delta_prefill_workspace_bytes(int seq_len, int num_v_heads, int head_k_dim,
                                            int head_v_dim);
void linear_delta_prefill(Context& ctx, Tensor& q, Tensor& k, Tensor& v, Tensor& a, Tensor& b,
                          Tensor* dt_bias, Tensor* A_log, Tensor& state, Tensor& out,
                          Tensor& workspace, int seq_len, int num_k_heads, int num_v_heads,
                          int head_k_dim, int head_v_dim, float eps, float scale);

// ---- Q/K preparation and the output gate (Ops.hpp:163-244) ----
// Multimodal position streams (interleaved mRoPE with pos_t/pos_h/pos_w) are
// not part of this path: the ops below throw when asked for them, and the
// decode variants also throw on a non-zero text_pos_delta that would apply
// (their rotary position and cache row are the same start_pos).

// Per-head RMSNorm in place (Ops.hpp:165-166): x [seq_len, num_heads*head_dim]
// bf16, weight [head_dim] bf16 (an invalid tensor means no weight).
void head_rms_norm(Context& ctx, Tensor& x, Tensor& weight, float eps, int seq_len, int num_heads,
                   int head_dim);

// output = input * sigmoid(gate), n bf16 elements (Ops.hpp:169-170);
// output may alias input.
void sigmoid_mul(Context& ctx, Tensor& input, Tensor& gate, Tensor& output, int n);

// NeoX RoPE in place over the full head (Ops.hpp:175-178) and over the first
// rotary_dim dims (Ops.hpp:181-194); rotary_dim is clamped to [2, head_dim]
// and made even. text_pos_delta shifts positions >= prompt_pos_len; with
// interleaved and all three of pos_t/pos_h/pos_w (device int arrays indexed by
// position) the frequency pairs take the mRoPE streams (ElementwiseOps.cpp:60-78).
// The decode-prepare ops below take the same arguments; their cache row stays
// start_pos.
void apply_rope(Context& ctx, Tensor& q, Tensor& k, int seq_len, int start_pos, int num_heads_q,
                int num_kv_heads, int head_dim, float theta);
void apply_rope_partial(Context& ctx, Tensor& q, Tensor& k, int seq_len, int start_pos, int num_heads_q,
                        int num_kv_heads, int head_dim, int rotary_dim, float theta,
                        bool interleaved = false, const int* pos_t = nullptr, const int* pos_h = nullptr,
                        const int* pos_w = nullptr, int prompt_pos_len = 0, int text_pos_delta = 0,
                        int mrope_section_t = 0, int mrope_section_h = 0, int mrope_section_w = 0);

// One-token QK-norm + RoPE + K/V append (Ops.hpp:205-211). q [1, Hq*D] and
// k [1, Hkv*D] are updated in place; the caches are [Hkv, max_seq, D]
// (max_seq from k_cache.shape(1)). Pair d rotates by start_pos * rope_freq[d]
// (f32 [head_dim/2]; the backends fill it with 1/theta^(2d/head_dim),
// Qwen3DenseBackend.cpp:232-236); an invalid rope_freq tensor uses theta.
void decode_prepare_qkv(Context& ctx, Tensor& q, Tensor& k, Tensor& v, Tensor& rope_freq,
                        Tensor& q_norm_weight, Tensor& k_norm_weight, Tensor& k_cache, Tensor& v_cache,
                        int start_pos, int num_heads_q, int num_kv_heads, int head_dim, float eps,
                        float theta);

// The same with a partial rotary width (Ops.hpp:216-230).
void decode_prepare_qkv_partial(Context& ctx, Tensor& q, Tensor& k, Tensor& v, Tensor& q_norm_weight,
                                Tensor& k_norm_weight, Tensor& k_cache, Tensor& v_cache, int start_pos,
                                int num_heads_q, int num_kv_heads, int head_dim, float eps, int rotary_dim,
                                float theta, bool interleaved = false, const int* pos_t = nullptr,
                                const int* pos_h = nullptr, const int* pos_w = nullptr,
                                int prompt_pos_len = 0, int text_pos_delta = 0, int mrope_section_t = 0,
                                int mrope_section_h = 0, int mrope_section_w = 0);

// Packed per-head q|gate [1, Hq*2D] split into q_out and gate_out [1, Hq*D],
// then as decode_prepare_qkv_partial (Ops.hpp:235-250).
void decode_prepare_qgkv_packed_partial(Context& ctx, Tensor& q_gate_packed, Tensor& k, Tensor& v,
                                        Tensor& q_out, Tensor& gate_out, Tensor& q_norm_weight,
                                        Tensor& k_norm_weight, Tensor& k_cache, Tensor& v_cache,
                                        int start_pos, int num_heads_q, int num_kv_heads, int head_dim,
                                        float eps, int rotary_dim, float theta, bool interleaved = false,
                                        const int* pos_t = nullptr, const int* pos_h = nullptr,
                                        const int* pos_w = nullptr, int prompt_pos_len = 0,
                                        int text_pos_delta = 0, int mrope_section_t = 0,
                                        int mrope_section_h = 0, int mrope_section_w = 0);

// ---- the whole Gated DeltaNet layer (conv ring, norms, recurrence, gate) ----
// Qwen35HybridTextBackend::run_linear_delta_decode_gpu (:975-1166) as a free
// function: qkv [1, 2*Hk*dk + Hv*dv], z [1, Hv*dv], a/b [1, Hv] bf16;
// conv1d_weight [conv_ch, conv_kernel] bf16 (Layer::linear_conv1d_weight);
// conv_state [conv_kernel-1, conv_ch] fp32 and state [Hv, dk, dv] fp32
// (LayerCache::linear_conv_state / linear_state) updated in place;
// norm_weight [dv] fp32; out [1, Hv*dv] bf16. conv_head is the cache's
// linear_conv_head and is advanced by one, as the backend does (:1163).
// scale = 1/sqrt(head_k_dim) as in the backend (:991). arrivals (s32
// [num_k_heads], zeroed once, left zero by every call) lets the layer run
// one workgroup per value head; null runs one per key head.
void linear_delta_layer_decode(Context& ctx, Tensor& qkv, Tensor& z, Tensor& a, Tensor& b, Tensor& conv1d_weight,
                               Tensor& conv_state, int& conv_head, Tensor* dt_bias, Tensor* A_log,
                               Tensor& norm_weight, Tensor& state, Tensor& out, int num_k_heads, int num_v_heads,
                               int head_k_dim, int head_v_dim, int conv_kernel, float eps,
                               Tensor* arrivals = nullptr);

// run_linear_delta_prefill_gpu_batched (:1306-1508): fused_all [seq_len,
// all_dim] rows of [qkv | z | a | b] (all_dim = conv_ch + Hv*dv + 2*Hv),
// out [seq_len, Hv*dv]; conv_head advanced by seq_len (:1506). workspace u8
// of at least linear_delta_layer_prefill_workspace_bytes(...).
size_t linear_delta_layer_prefill_workspace_bytes(int seq_len, int num_k_heads, int num_v_heads, int head_k_dim,
                                                  int head_v_dim);
void linear_delta_layer_prefill(Context& ctx, Tensor& fused_all, Tensor& out, int seq_len, Tensor& conv1d_weight,
                                Tensor& conv_state, int& conv_head, Tensor* dt_bias, Tensor* A_log,
                                Tensor& norm_weight, Tensor& state, Tensor& workspace, int num_k_heads,
                                int num_v_heads, int head_k_dim, int head_v_dim, int conv_kernel, float eps);

}  // namespace ops

/*
 * aila_hip.h - C ABI of the MI355X (gfx950) attention hot path for Aila.
 *
 * Every entry point is asynchronous on the given HIP stream (`stream` is a
 * hipStream_t passed as void*, NULL = the default stream), allocates nothing
 * and returns 0 on success or a negative AILA_HIP_* code. On failure the
 * message is available from aila_hip_last_error() (thread-local).
 *
 * Pointers are device pointers unless stated otherwise. bf16 tensors are
 * passed as void* to 16-bit bf16 storage; fp32 as float*. All tensors are
 * dense row-major with the shapes given below.
 *
 * Reference interfaces replaced (Aila, SYCL): namespace ops in
 * src/ops/Ops.hpp and the DeltaNet member functions of
 * src/models/Qwen35HybridTextBackend.hpp.
 */
#ifndef AILA_HIP_H
#define AILA_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  AILA_HIP_OK = 0,
  AILA_HIP_EINVAL = -1,       /* bad shape / pointer / size */
  AILA_HIP_EUNSUPPORTED = -2, /* shape outside the compiled kernel set */
  AILA_HIP_ELAUNCH = -3,      /* HIP runtime error at launch */
  AILA_HIP_EWORKSPACE = -4    /* workspace missing or too small */
};

/* Last error message of the calling thread ("" if none). */
const char* aila_hip_last_error(void);
/* ABI version: (major << 16) | minor. */
int aila_hip_version(void);

/* Rotary positions of a token when they differ from its cache row: the text
 * position shift and the interleaved multimodal RoPE (mRoPE) streams of
 * ops::apply_rope_partial / decode_prepare_qkv_partial /
 * decode_prepare_qgkv_packed_partial (src/ops/ElementwiseOps.cpp:33-103,
 * 555-863). For the token in cache row r of sequence b, with
 * P = prompt_pos_lens ? prompt_pos_lens[b] : prompt_pos_len and
 * delta = text_pos_deltas ? text_pos_deltas[b] : text_pos_delta:
 *   scalar = r >= P ? r + delta : r                       (:54-58)
 * and frequency index d (0 <= d < rotary_dim/2) rotates at `scalar`, or, when
 * `interleaved` is nonzero and pos_t, pos_h and pos_w are all given, at
 *   h-stream if d % 3 == 1 and d / 3 < mrope_section_h,
 *   w-stream if d % 3 == 2 and d / 3 < mrope_section_w,
 *   t-stream otherwise                                    (:60-78)
 * where a stream's value is pos_X[b * pos_stride + r] for r < P and `scalar`
 * past the prompt. pos_t/pos_h/pos_w are device int arrays holding at least
 * P entries per sequence; mrope_section_t is accepted and, as in the
 * reference, unused. A zero-initialised struct (or a NULL pointer where an
 * entry point takes one) means "rotate at the cache row". The cache row a
 * decode step appends to is never shifted.
 * inv_freq (optional device float[rotary_dim/2]): pair d rotates by
 * position * inv_freq[d] instead of position * theta^(-2d/rotary_dim) -- the
 * backend's precomputed rope_freq table of ops::decode_prepare_qkv
 * (ElementwiseOps.cpp:105-216, angle = start_pos * rope_freq[d]). */
typedef struct aila_hip_rope_pos {
  int interleaved;
  const int* pos_t;
  const int* pos_h;
  const int* pos_w;
  int pos_stride;
  int prompt_pos_len;
  int text_pos_delta;
  const int* prompt_pos_lens; /* optional device int[B] */
  const int* text_pos_deltas; /* optional device int[B] */
  int mrope_section_t, mrope_section_h, mrope_section_w;
  const float* inv_freq;      /* optional device float[rotary_dim/2] */
} aila_hip_rope_pos;

/* ---------------------------------------------------------------- GQA --- */

/* Workspace bytes needed by aila_hip_gqa_decode for up to B sequences of
 * Hq heads of head_dim D (split-K partial records). */
size_t aila_hip_gqa_decode_workspace_size(int B, int Hq, int D);

/* Single-token GQA decode over a bf16 KV cache (split-K flash-decode).
 * Replaces ops::attention_decode (src/ops/Ops.hpp:264-269;
 * src/ops/AttentionOps.cpp:499-643) and its kernels (:73-320).
 *   q        [B, Hq, D] bf16        out [B, Hq, D] bf16
 *   k_cache  [B, Hkv, max_seq, D] bf16, v_cache likewise
 *            (per sequence the reference layout [Hkv, max_seq, D],
 *             src/memory/KVCache.hpp:9-45)
 *   cached_len  keys [0, cached_len) are attended (all sequences), or
 *   seq_lens    optional device int[B]: sequence b attends
 *               [0, min(seq_lens[b], cached_len)); a length of 0 yields 0.
 *   workspace   >= aila_hip_gqa_decode_workspace_size(B, Hq, D) bytes, or
 *               NULL for the single-pass variant (one workgroup per head
 *               group, no split; slower for long contexts).
 * Head h reads KV head h / (Hq / Hkv). Softmax scale 1/sqrt(D).
 * Supported: D in {64, 128, 256}, any integer Hq/Hkv (ratios 1, 2, 4 and 8
 * map onto the kernel's query-head tile exactly; others run on the next
 * larger tile, and ratios above 8 on ceil(ratio / 8) workgroups per KV
 * head, each streaming that head's K/V).
 * Bandwidth note: a head stride max_seq*D*2 that is a multiple of 256 KiB
 * (e.g. max_seq a multiple of 512 rows at D = 256) streams at full rate;
 * an odd row count measured ~7% slower on MI355X. */
int aila_hip_gqa_decode(const void* q, const void* k_cache, const void* v_cache,
                        void* out, void* workspace, size_t workspace_bytes,
                        int B, int Hq, int Hkv, int D, int max_seq,
                        int cached_len, const int* seq_lens, void* stream);

/* The same decode over a window of each sequence's cache with attention
 * sinks: the AILA_ATTN_DECODE_WINDOW / _WINDOW_START / _SINK knobs of
 * ops::attention_decode (src/ops/AttentionOps.cpp:533-551, 598-616, and the
 * tail_start / sink_len row map of :73-166, 168-320). A sequence of L rows
 * with L > window_start attends rows [0, s) and [L - w, L), where
 * w = min(L, window) and s = min(sink, L - w); when s + w >= L, or window = 0,
 * or L <= window_start, it attends all L rows. window_start < 0 means
 * max(512, window), the reference's default. L is cached_len, or
 * min(seq_lens[b], cached_len) per sequence. Other arguments and results as
 * aila_hip_gqa_decode; rows outside the window are never read. */
int aila_hip_gqa_decode_window(const void* q, const void* k_cache, const void* v_cache,
                               void* out, void* workspace, size_t workspace_bytes,
                               int B, int Hq, int Hkv, int D, int max_seq,
                               int cached_len, const int* seq_lens, int window,
                               int window_start, int sink, void* stream);

/* GQA decode over a paged KV cache. The reference keeps one contiguous
 * [Hkv, max_seq, D] cache per sequence (src/memory/KVCache.hpp:9-45) and
 * has no paged layout; this is the paged option of the same decode
 * (ops::attention_decode, src/ops/AttentionOps.cpp:499-643) for serving
 * engines that allocate the cache in fixed-size pages.
 *   k_pages, v_pages  [num_pages, Hkv, page_size, D] bf16 page pool
 *   block_table       device int[B, max_pages]: row t of sequence b is row
 *                     t % page_size of page block_table[b*max_pages + t/page_size].
 *                     Entries covering rows < seq_lens[b] must index the pool
 *                     (the kernel dereferences only those); the rest, e.g. -1
 *                     for unallocated pages, are never used as addresses.
 *   seq_lens          device int[B] (required): sequence b attends rows
 *                     [0, min(seq_lens[b], max_len))
 *   max_len           host bound on every seq_lens[b] (<= max_pages*page_size);
 *                     it sizes the split plan as cached_len does.
 *   page_size         a multiple of 16.
 * Other arguments, the workspace and the results as aila_hip_gqa_decode
 * (identical results for identical rows). */
int aila_hip_gqa_decode_paged(const void* q, const void* k_pages,
                              const void* v_pages, void* out, void* workspace,
                              size_t workspace_bytes, int B, int Hq, int Hkv,
                              int D, int page_size, const int* block_table,
                              int max_pages, int max_len, const int* seq_lens,
                              void* stream);

/* Append one token's K/V row per sequence into its page: k_new/v_new
 * [B, Hkv, D] bf16 go to row positions[b] (device int[B]) of sequence b in
 * the paged layout of aila_hip_gqa_decode_paged. Positions outside
 * [0, max_pages*page_size) are skipped; the table entry of every other
 * position must index the pool. (The paged counterpart of the cache
 * write of ops::decode_prepare_qkv, src/ops/ElementwiseOps.cpp:105-216.) */
int aila_hip_kv_append_paged(const void* k_new, const void* v_new,
                             void* k_pages, void* v_pages, int B, int Hkv,
                             int D, int page_size, const int* block_table,
                             int max_pages, const int* positions, void* stream);

/* Allocation-free variant of aila_hip_gqa_decode. No counterpart in the
 * reference: it is for callers that cannot allocate device memory or pass a
 * workspace (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). The split records live in a static device array
 * of aila_hip_gqa_decode_noalloc_max_bytes() bytes (8 MiB) per GPU, held
 * until the process ends; it calls no allocating routine. Sizes whose two
 * split records per head exceed it (B*Hq*2*(16+D)*4 bytes > 8 MiB) are
 * rejected with AILA_HIP_EINVAL. Every call on one GPU shares that array,
 * so calls that overlap in time on the same GPU (different streams, or
 * different threads) race: serialise them. Arguments and results as
 * aila_hip_gqa_decode with a workspace. */
size_t aila_hip_gqa_decode_noalloc_max_bytes(void);
int aila_hip_gqa_decode_noalloc(const void* q, const void* k_cache,
                                const void* v_cache, void* out, int B, int Hq,
                                int Hkv, int D, int max_seq, int cached_len,
                                const int* seq_lens, void* stream);

/* Decode step with the new token's K/V append fused in (the cache write of
 * ops::decode_prepare_qkv, src/ops/ElementwiseOps.cpp:105-216, followed by
 * ops::attention_decode with cached_len = start_pos + 1, as the backends call
 * them at Qwen35HybridTextBackend.cpp:2109 and :2176).
 *   k_new/v_new [B, Hkv, D] bf16 are written to cache row `pos` of every
 *   sequence (or row positions[b] when the optional device int[B]
 *   `positions` is given; then every positions[b] must be <= pos, which only
 *   sizes the launch), and sequence b attends rows [0, row].
 * Other arguments as aila_hip_gqa_decode. */
int aila_hip_gqa_decode_append(const void* q, const void* k_new,
                               const void* v_new, void* k_cache,
                               void* v_cache, void* out, void* workspace,
                               size_t workspace_bytes, int B, int Hq, int Hkv,
                               int D, int max_seq, int pos,
                               const int* positions, void* stream);

/* The whole attention decode step of a GQA layer in one split-K launch:
 * ops::decode_prepare_qkv_partial / decode_prepare_qgkv_packed_partial
 * (src/ops/ElementwiseOps.cpp:555-863: per-head RMSNorm of q and k rounded to
 * bf16, NeoX RoPE over the first rotary_dim dims at the token's position
 * rounded to bf16, K/V append) followed by ops::attention_decode, as the
 * hybrid backend calls them (Qwen35HybridTextBackend.cpp:2109-2180).
 *   q_in [B, Hq, D] bf16 (packed_gate 0), or [B, Hq, 2D] q|gate per head:
 *   packed_gate 1 copies the gate half to gate_out [B, Hq, D]; packed_gate
 *   2 applies it instead, out = attention * sigmoid(gate) (the gated
 *   attention epilogue ops::sigmoid_mul, ElementwiseOps.cpp:519-553, in the
 *   same launch; gate_out unused); k_new/v_new
 *   [B, Hkv, D]; q_norm_w/k_norm_w [D] bf16 or NULL (weight 1). The prepared
 *   k and v_new go to cache row pos (or positions[b]) and sequence b attends
 *   rows [0, row]; q_in and k_new are not modified (the prepared q lives only
 *   in LDS). rotary_dim is clamped to [2, D] and made even. rope_pos (NULL =
 *   rotate at the cache row) gives the text shift / mRoPE positions of
 *   aila_hip_rope_pos; the new row is still written at the cache row. Other
 *   arguments as aila_hip_gqa_decode. */
int aila_hip_gqa_decode_prepare_append(const void* q_in, int packed_gate,
                                       void* gate_out, const void* k_new,
                                       const void* v_new, const void* q_norm_w,
                                       const void* k_norm_w, void* k_cache,
                                       void* v_cache, void* out,
                                       void* workspace, size_t workspace_bytes,
                                       int B, int Hq, int Hkv, int D,
                                       int max_seq, int rotary_dim, float theta,
                                       float eps, int pos, const int* positions,
                                       const aila_hip_rope_pos* rope_pos,
                                       void* stream);

/* Append one decoded token's K and V per sequence to the cache (the
 * cache-write half of ops::decode_prepare_qkv, src/ops/ElementwiseOps.cpp:
 * 105-216, without the norm/RoPE): k_new/v_new [B, Hkv, D] bf16 ->
 * k_cache/v_cache [B, Hkv, max_seq, D] row `pos`, or row positions[b] when
 * the optional device int[B] `positions` is given (rows outside
 * [0, max_seq) are skipped). Requires D % 8 == 0. */
int aila_hip_kv_append(const void* k_new, const void* v_new, void* k_cache,
                       void* v_cache, int B, int Hkv, int D, int max_seq,
                       int pos, const int* positions, void* stream);

/* Causal GQA prefill over the current chunk on bf16 MFMA (flash attention).
 * Replaces ops::attention_prefill (src/ops/Ops.hpp:278-282;
 * src/ops/AttentionOps.cpp:649-842) fused with the two ops::copy_to_cache
 * calls that precede it in the backends (Ops.hpp:199-201,
 * AttentionOps.cpp:2513-2532; Qwen3DenseBackend.cpp:318-325).
 *   q [S, Hq*D], k/v [S, Hkv*D] bf16 (token-major, already QK-normed/RoPE'd)
 *   out [S, Hq*D] bf16; query i attends keys [0, i].
 *   k_cache/v_cache [Hkv, max_seq, D] bf16 or both NULL: when given, k/v are
 *   also written to cache rows [cache_pos, cache_pos + S).
 * Supported: D in {64, 128, 256}, Hq % Hkv == 0. */
int aila_hip_gqa_prefill(const void* q, const void* k, const void* v, void* out,
                         void* k_cache, void* v_cache, int cache_pos,
                         int max_seq, int S, int Hq, int Hkv, int D,
                         void* stream);

/* Incremental (cached) prefill: replaces ops::attention_prefill_cached
 * (src/ops/Ops.hpp:293-298; src/ops/AttentionOps.cpp:2308-2507).
 *   q [S, Hq*D]; k_cache/v_cache [Hkv, max_seq, D] already holding rows
 *   [0, start_pos + S); query i (position start_pos + i) attends cache rows
 *   [0, start_pos + i]. out [S, Hq*D] bf16. */
int aila_hip_gqa_prefill_cached(const void* q, const void* k_cache,
                                const void* v_cache, void* out, int S,
                                int start_pos, int Hq, int Hkv, int D,
                                int max_seq, void* stream);

/* The same prefill with a workspace, for a short turn over a long cached
 * prefix: when the (query block pair, head) grid would leave the device
 * mostly idle, each query block's keys are cut into runs walked by separate
 * workgroups, whose partial softmax states {m, l, acc} (fp32, D + 4 floats
 * per row and run) meet in a merge pass. The reference passes its score
 * buffer scores_buf [heads, seq, total] fp32 here (ops::attention_prefill_cached,
 * src/ops/Ops.hpp:293-298), which is far larger than the records need.
 * workspace_size returns the bytes for the run count this call would use
 * (0: no split); a smaller workspace gives fewer runs, a null one none.
 * Results as aila_hip_gqa_prefill_cached within the attention tolerance
 * (the runs' sums are added in another order). */
size_t aila_hip_gqa_prefill_cached_workspace_size(int S, int start_pos,
                                                  int Hq, int Hkv, int D);
int aila_hip_gqa_prefill_cached_ws(const void* q, const void* k_cache,
                                   const void* v_cache, void* out,
                                   void* workspace, size_t workspace_bytes,
                                   int S, int start_pos, int Hq, int Hkv,
                                   int D, int max_seq, void* stream);

/* ops::copy_to_cache (src/ops/Ops.hpp:199-201; AttentionOps.cpp:2513-2532):
 * new_kv [S, H*D] bf16 -> cache [H, max_seq, D] rows [start_pos, start_pos+S).
 * Requires D % 8 == 0 and 16-byte aligned pointers. */
int aila_hip_copy_to_cache(const void* new_kv, void* cache, int S,
                           int start_pos, int H, int D, int max_seq,
                           void* stream);

/* ----------------------------------------------------------- DeltaNet --- */

/* One Gated DeltaNet decode step (the recurrence of
 * Qwen35HybridTextBackend::run_linear_delta_decode_gpu,
 * src/models/Qwen35HybridTextBackend.cpp:975-1166, host form :1729-1780),
 * for B independent sequences, after conv1d/SiLU:
 *   q, k [B, Hk, dk] bf16 (L2-normalised in-kernel: x / sqrt(sum x^2 + eps))
 *   v    [B, Hv, dv] bf16; a, b [B, Hv] bf16
 *   beta = sigmoid(b), decay = exp(-softplus(a + dt_bias) * exp(A_log))
 *   dt_bias [Hv] bf16 and A_log [Hv] fp32 may be NULL (0).
 *   state [B, Hv, dk, dv] fp32, S[j*dv + i], updated in place:
 *     S *= decay; u = S^T k; d = (v - u) * beta; S += k d^T
 *   out  [B, Hv, dv] bf16 = (S^T q) * scale.
 * Value head hv uses key head hv / (Hv / Hk) (clamp(hv, 0, Hk - 1) when Hk
 * does not divide Hv, as Qwen35HybridTextBackend.cpp:104-118). The state is
 * read once and written once. Tuned kernels: dk in {64, 128, 256}, dv a
 * multiple of 4, Hk dividing Hv; other shapes with dk, dv <= 256 run a
 * general-shape kernel (one workgroup per value head and sequence, state
 * in global memory, same math). */
int aila_hip_deltanet_decode(const void* q, const void* k, const void* v,
                             const void* a, const void* b,
                             const void* dt_bias, const float* A_log,
                             float* state, void* out, int B, int Hk, int Hv,
                             int dk, int dv, float eps, float scale,
                             void* stream);

/* The whole Gated DeltaNet layer for one token per sequence, between the
 * input projection and o_proj (the fast path of
 * Qwen35HybridTextBackend::run_linear_delta_decode_gpu,
 * src/models/Qwen35HybridTextBackend.cpp:1013-1166; host form :1640-1798):
 *   qkv  row b at qkv + b*qkv_stride: [q (Hk*dk) | k (Hk*dk) | v (Hv*dv)] bf16
 *   conv: y_c = silu(ring[h][c] w[c,0] + ring[h+1][c] w[c,1]
 *                    + ring[h+2][c] w[c,2] + x_c w[c,3])   (rows mod 3)
 *         then ring[h][c] = x_c, where h = conv_heads ? conv_heads[b] : conv_head;
 *         conv_w [ch, 4] bf16; conv_state [B, 3, ch] fp32, ch = 2*Hk*dk + Hv*dv.
 *         The caller advances the head by one per step (as :1163 does).
 *   recurrence: as aila_hip_deltanet_decode on the fp32 conv outputs;
 *         a, b at a + b*ab_stride + hv (ab_stride = Hv for separate tensors,
 *         the fused row width for the backend's [qkv | z | a | b] row).
 *   gate: out[b, hv, :] = bf16(rmsnorm(o) * norm_w * silu(z)), rmsnorm over dv,
 *         z row b at z + b*z_stride, norm_w [dv] fp32 (:1153-1160, :153-173).
 * state [B, Hv, dk, dv] fp32 is read and written once. Tuned kernels: dk =
 * dv = 128, conv kernel 4, Hv / Hk in {1, 2, 4} (the reference fast path's
 * shapes). Other shapes (dk, dv <= 256, conv kernel 1..16, any head counts,
 * key head as aila_hip_deltanet_decode) run the general-shape kernel, the
 * role of the reference's generic fallback (:1168-1304), followed by a
 * ring-rewrite launch; conv_state is then [B, K-1, ch] and arrivals is
 * ignored.
 *   arrivals  optional device uint32[B*Hk], zero before the first call and
 *             left zero by every call: with it (and Hv > Hk) the layer runs
 *             one workgroup per value head instead of one per key head (the
 *             key head's workgroups count their reads of the shared q/k ring
 *             row in it, and the last one replaces that row). Calls that
 *             overlap in time must not share one array. NULL: one workgroup
 *             per key head. Same results either way. */
int aila_hip_deltanet_layer_decode(const void* qkv, int qkv_stride,
                                   const void* z, int z_stride, const void* a,
                                   const void* b, int ab_stride,
                                   const void* conv_w, float* conv_state,
                                   int conv_head, const int* conv_heads,
                                   const void* dt_bias, const float* A_log,
                                   const float* norm_w, float* state,
                                   void* out, int B, int Hk, int Hv, int dk,
                                   int dv, int conv_kernel, float eps,
                                   float scale, unsigned int* arrivals,
                                   void* stream);

/* Workspace bytes for aila_hip_deltanet_layer_prefill: the per-chunk
 * records (as aila_hip_deltanet_prefill's, plus the key residual; about
 * 121 KiB per sequence, value head and 64-token chunk). 0 for the shapes
 * that run the general-shape kernel (no workspace needed). */
size_t aila_hip_deltanet_layer_prefill_workspace_size(int B, int T, int Hk,
                                                      int Hv, int dk, int dv);

/* The whole Gated DeltaNet layer over T tokens per sequence (the fast path
 * of Qwen35HybridTextBackend::run_linear_delta_prefill_gpu_batched,
 * src/models/Qwen35HybridTextBackend.cpp:1306-1508, which runs the decode
 * step token by token; host form :1640-1798). Token t of sequence b reads
 * qkv + (b*T + t)*qkv_stride, z + (b*T + t)*z_stride and a/b +
 * (b*T + t)*ab_stride + hv (so the backend's fused [qkv | z | a | b] row is
 * qkv = row, z = row + ch, a = row + ch + Hv*dv, b = a + Hv, every stride the
 * row width). Same math as aila_hip_deltanet_layer_decode applied to the
 * tokens in order, with the ring head advanced per token; the caller
 * advances its head by T afterwards (:1506). The chunk prep forms the conv
 * + SiLU of its rows itself and carries it fp32-accurate (bf16 hi +
 * residual) into the recurrence, which runs chunked as
 * aila_hip_deltanet_prefill; the last pass applies the gated RMSNorm and
 * rewrites the ring. out [B, T, Hv*dv] bf16. Chunked path: dk = dv = 128,
 * conv kernel 4, Hv % Hk == 0; qkv 8-byte aligned with qkv_stride a
 * multiple of 4 (a sequence whose rows span 2 GiB or more runs as
 * consecutive segments of whole 64-token chunks inside the call, with the
 * same results). Other shapes (dk, dv <= 256,
 * conv kernel 1..16, any head counts) run the general-shape kernel token by
 * token, as the reference's batched prefill does; no workspace. */
int aila_hip_deltanet_layer_prefill(const void* qkv, int qkv_stride,
                                    const void* z, int z_stride, const void* a,
                                    const void* b, int ab_stride,
                                    const void* conv_w, float* conv_state,
                                    int conv_head, const void* dt_bias,
                                    const float* A_log, const float* norm_w,
                                    float* state, void* out, void* workspace,
                                    size_t workspace_bytes, int B, int T,
                                    int Hk, int Hv, int dk, int dv,
                                    int conv_kernel, float eps, float scale,
                                    void* stream);

/* Workspace bytes for aila_hip_deltanet_prefill (per-chunk W and its
 * residual, U, P, Q, K^T and decay factors, in the scan's operand order;
 * 105 KiB per (sequence, value head, 64-token chunk), of which the key
 * head's K^T and Q parts are used once per key head). 0 for the shapes that
 * run the general-shape kernel. */
size_t aila_hip_deltanet_prefill_workspace_size(int B, int T, int Hv, int dk,
                                                int dv);

/* Chunked Gated DeltaNet prefill (chunk 64, WY/UT form on bf16 MFMA): the
 * recurrence of aila_hip_deltanet_decode applied to T tokens, replacing the
 * token-sequential Qwen35HybridTextBackend::run_linear_delta_prefill_gpu_batched
 * (src/models/Qwen35HybridTextBackend.cpp:1306-1508) after conv1d/SiLU.
 *   q, k [B, T, Hk, dk] bf16; v [B, T, Hv, dv] bf16; a, b [B, T, Hv] bf16
 *   dt_bias [Hv] bf16 / A_log [Hv] fp32 may be NULL
 *   state [B, Hv, dk, dv] fp32: initial state in, final state out
 *   out [B, T, Hv, dv] bf16
 * Chunked path: dk = dv = 128 with Hk dividing Hv; other shapes (dk, dv <=
 * 256) run the general-shape kernel token by token (no workspace). */
int aila_hip_deltanet_prefill(const void* q, const void* k, const void* v,
                              const void* a, const void* b,
                              const void* dt_bias, const float* A_log,
                              float* state, void* out, void* workspace,
                              size_t workspace_bytes, int B, int T, int Hk,
                              int Hv, int dk, int dv, float eps, float scale,
                              void* stream);

/* ------------------------------------ QK-norm, RoPE, gate (GQA layer) --- */

/* Decode-step preparation for B sequences (one token each): per-head RMSNorm
 * of q and k (weights q_norm_w / k_norm_w [D] bf16, NULL = 1), NeoX
 * half-split RoPE on the first rotary_dim dims (angle = position *
 * theta^(-2d/rotary_dim)), and k/v appended to the caches at the position.
 * Replaces ops::decode_prepare_qkv (src/ops/ElementwiseOps.cpp:105-216),
 * ops::decode_prepare_qkv_partial (:555-705) and
 * ops::decode_prepare_qgkv_packed_partial (:707-863, packed_gate != 0) for
 * the cache row as the position, or the shifted / mRoPE positions of
 * rope_pos (NULL = the cache row); rounding points as the reference (bf16
 * after the norm and after the rotation).
 *   q_in     [B, Hq, D] bf16, or [B, Hq, 2D] (q | gate per head) if packed_gate
 *   q_out    [B, Hq, D] bf16 (may equal q_in when not packed)
 *   gate_out [B, Hq, D] bf16, the gate half copied through (packed_gate only)
 *   k        [B, Hkv, D] bf16, normalised and rotated in place
 *   v        [B, Hkv, D] bf16
 *   k_cache/v_cache [B, Hkv, max_seq, D] bf16 or both NULL (no append)
 *   position of sequence b: positions[b] (device int[B]) if given, else pos.
 * Supported: D in {64, 128, 256}. */
int aila_hip_decode_prepare_qkv(const void* q_in, int packed_gate, void* q_out, void* gate_out,
                                void* k, const void* v, const void* q_norm_w, const void* k_norm_w,
                                void* k_cache, void* v_cache, int B, int Hq, int Hkv, int D,
                                int max_seq, int rotary_dim, float theta, float eps, int pos,
                                const int* positions, const aila_hip_rope_pos* rope_pos,
                                void* stream);

/* Per-head RMSNorm in place over x [S, H, D] bf16 with weight [D] bf16 (NULL
 * = 1). Replaces ops::head_rms_norm (src/ops/NormOps.cpp:277-321).
 * Supported: D in {64, 128, 256}. */
int aila_hip_head_rms_norm(void* x, const void* weight, int S, int H, int D, float eps, void* stream);

/* RoPE in place on q [S, Hq, D] and k [S, Hkv, D] bf16, NeoX half-split
 * over the first rotary_dim dims; row s is the token in cache row
 * start_pos + s, rotated at that row or at the positions rope_pos gives for
 * it (sequence 0 of aila_hip_rope_pos; NULL = the row). Replaces
 * ops::apply_rope / apply_rope_partial, including the text shift and the
 * interleaved mRoPE streams (src/ops/ElementwiseOps.cpp:33-103).
 * Supported: D in {64, 128, 256}, Hkv <= Hq. */
int aila_hip_apply_rope(void* q, void* k, int S, int start_pos, int Hq, int Hkv, int D, int rotary_dim,
                        float theta, const aila_hip_rope_pos* rope_pos, void* stream);

/* output = input * sigmoid(gate), n bf16 elements (output may equal input).
 * Replaces ops::sigmoid_mul (src/ops/ElementwiseOps.cpp:519-553), the
 * gated-attention output gate. */
int aila_hip_sigmoid_mul(const void* input, const void* gate, void* output, long n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AILA_HIP_H */

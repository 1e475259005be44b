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
 * Supported: D in {64, 128, 256}, Hq/Hkv in {1, 2, 4, 8}. */
int aila_hip_gqa_decode(const void* q, const void* k_cache, const void* v_cache,
                        void* out, void* workspace, size_t workspace_bytes,
                        int B, int Hq, int Hkv, int D, int max_seq,
                        int cached_len, const int* seq_lens, void* stream);

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
 * Value head hv uses key head hv / (Hv / Hk). The state is read once and
 * written once. Supported: dk in {64, 128, 256}, dv a multiple of 4. */
int aila_hip_deltanet_decode(const void* q, const void* k, const void* v,
                             const void* a, const void* b,
                             const void* dt_bias, const float* A_log,
                             float* state, void* out, int B, int Hk, int Hv,
                             int dk, int dv, float eps, float scale,
                             void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AILA_HIP_H */

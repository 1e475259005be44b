// General-shape Gated DeltaNet (sequential over tokens, one workgroup per
// value head and sequence); used by the DeltaNet entry points for the shapes
// their tuned kernels do not compile.
#pragma once

#include "common.hpp"

namespace aila {

struct GenericDeltaNet {
  int layer;                 // 0: recurrence on q, k, v; 1: the whole layer
  // recurrence inputs: q, k [B, T, Hk, dk], v [B, T, Hv, dv] bf16
  const bf16* q;
  const bf16* k;
  const bf16* v;
  // layer inputs: token (b, t) rows at qkv + (b*T + t)*qkv_stride
  // ([q | k | v], ch = 2*Hk*dk + Hv*dv) and z + (b*T + t)*z_stride
  const bf16* qkv;
  long qkv_stride;
  const bf16* z;
  long z_stride;
  const bf16* conv_w;        // [ch, K] bf16
  float* conv_state;         // [B, K-1, ch] fp32 ring
  int conv_head;
  const int* conv_heads;     // optional device int[B]
  int K;                     // conv kernel width (layer only)
  const float* norm_w;       // [dv] fp32 (layer only)
  // gates: a, b of token (b, t), value head hv at + (b*T + t)*ab_stride + hv
  const bf16* a;
  const bf16* b;
  long ab_stride;
  const bf16* dt_bias;       // [Hv] or null
  const float* A_log;        // [Hv] or null
  float* state;              // [B, Hv, dk, dv] fp32, S[j*dv + i]
  bf16* out;                 // [B, T, Hv, dv] bf16
  int B, T, Hk, Hv, dk, dv;
  float eps, scale;
};

// dk, dv <= 256 and conv kernel width <= 16.
bool deltanet_generic_fits(int dk, int dv, int K);
// Launches the sequential kernel (and, for the layer, the ring rewrite).
int deltanet_generic_launch(const GenericDeltaNet& p, hipStream_t st, const char* what);

}  // namespace aila

// Per-head QK-norm + RoPE + K/V append (decode), the prefill-side norm and
// RoPE, and the gated-attention sigmoid multiply.
//
// Reference: ops::decode_prepare_qkv / _partial / decode_prepare_qgkv_packed_partial
// (src/ops/ElementwiseOps.cpp:105-216, 555-705, 707-863), ops::head_rms_norm
// (src/ops/NormOps.cpp:277-321), ops::apply_rope_partial (ElementwiseOps.cpp
// :33-103) and ops::sigmoid_mul (:519-553). The rounding points are the
// reference's: the normalised head is rounded to bf16, RoPE reads the
// rounded values and rounds again; dims past the rotary width keep the
// normalised value. Rotation is NeoX half-split over the first `rot` dims,
// angle = position * theta^(-2d/rot).
//
// Batched (the reference has one sequence): q [B, Hq, D] (or packed q|gate
// [B, Hq, 2D]), k/v [B, Hkv, D], caches [B, Hkv, max_seq, D]; the position of
// sequence b is `pos` or positions[b] (device), so a step can replay from a
// HIP graph. One wave per (head, sequence); the rotation partner d + rot/2
// may sit in another lane, so the rounded normalised head goes through LDS.
#include "common.hpp"

#include <algorithm>
#include <type_traits>

namespace aila {
namespace {

__device__ __forceinline__ float wave_sum64(float x) { return wave_sum(x); }

// Normalise one head (D values, lanes own d = lane + 64 i) into LDS as the
// bf16-rounded value, and return nothing; `w` may be null (weight 1).
template <int D>
__device__ __forceinline__ void norm_head_to_lds(const bf16* __restrict__ x, const bf16* __restrict__ w, float eps,
                                                 float* s_row) {
  constexpr int E = D / 64;
  const int lane = threadIdx.x & 63;
  float v[E], ss = 0.f;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    v[i] = bf2f(x[lane + 64 * i]);
    ss = fmaf(v[i], v[i], ss);
  }
  ss = wave_sum64(ss);
  const float rms = sqrtf(ss / static_cast<float>(D) + eps);
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int d = lane + 64 * i;
    const float wd = w ? bf2f(w[d]) : 1.0f;
    s_row[d] = bf2f(f2bf((v[i] / rms) * wd));
  }
}

// RoPE from the rounded normalised head in LDS to `y` (bf16); frequency
// index j rotates at rope_freq_pos(rp, j) (the row's position, or its mRoPE
// stream).
template <int D>
__device__ __forceinline__ void rope_from_lds(const float* s_row, bf16* __restrict__ y, int rot, RowPos rp,
                                              const RopePos& rpos, const RopeFreq& rf) {
  constexpr int E = D / 64;
  const int lane = threadIdx.x & 63;
  const int half = rot / 2;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int d = lane + 64 * i;
    float r = s_row[d];
    if (d < rot) {
      const int dd = d < half ? d : d - half;                 // frequency index
      const float freq = rope_inv_freq(rpos, rf, dd);
      const float ang = rope_freq_pos(rp, dd) * freq;
      const float c = cosf(ang), s = sinf(ang);
      r = d < half ? s_row[d] * c - s_row[d + half] * s : s_row[d] * c + s_row[d - half] * s;
    }
    y[d] = f2bf(r);
  }
}

template <int D>
__global__ __launch_bounds__(64) void decode_prep_kernel(
    const bf16* __restrict__ q_in, int q_in_stride, bf16* __restrict__ q_out, bf16* __restrict__ gate_out,
    bf16* __restrict__ k, const bf16* __restrict__ v, const bf16* __restrict__ qn_w,
    const bf16* __restrict__ kn_w, bf16* __restrict__ k_cache, bf16* __restrict__ v_cache, int Hq, int Hkv,
    int max_seq, int rot, RopeFreq rf, float eps, int pos, const int* __restrict__ positions, RopePos ropep) {
  __shared__ float s_row[D];
  const int hh = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x;
  const int p = positions ? positions[b] : pos;
  const RowPos rp = rope_row_pos(ropep, b, p);
  if (hh < Hq) {
    const bf16* src = q_in + (static_cast<size_t>(b) * Hq + hh) * q_in_stride;
    bf16* dst = q_out + (static_cast<size_t>(b) * Hq + hh) * D;
    if (gate_out) {   // packed q|gate: the gate half is copied through
      bf16* g = gate_out + (static_cast<size_t>(b) * Hq + hh) * D;
      for (int d = lane; d < D; d += 64) g[d] = src[D + d];
    }
    norm_head_to_lds<D>(src, qn_w, eps, s_row);
    __syncthreads();
    rope_from_lds<D>(s_row, dst, rot, rp, ropep, rf);
    return;
  }
  const int h = hh - Hq;
  bf16* kr = k + (static_cast<size_t>(b) * Hkv + h) * D;
  norm_head_to_lds<D>(kr, kn_w, eps, s_row);
  __syncthreads();
  rope_from_lds<D>(s_row, kr, rot, rp, ropep, rf);
  if (k_cache && p >= 0 && p < max_seq) {
    // each lane re-reads only the elements it wrote itself
    const size_t row = ((static_cast<size_t>(b) * Hkv + h) * max_seq + p) * D;
    const bf16* vr = v + (static_cast<size_t>(b) * Hkv + h) * D;
    for (int d = lane; d < D; d += 64) {
      k_cache[row + d] = kr[d];
      v_cache[row + d] = vr[d];
    }
  }
}

// head_rms_norm over rows of D: one wave per row, in place.
template <int D>
__global__ __launch_bounds__(64) void head_rms_norm_kernel(bf16* __restrict__ x, const bf16* __restrict__ w,
                                                          float eps, long rows) {
  __shared__ float s_row[D];
  const long r = blockIdx.x + static_cast<long>(gridDim.x) * blockIdx.y;
  if (r >= rows) return;
  bf16* xr = x + r * D;
  norm_head_to_lds<D>(xr, w, eps, s_row);
  const int lane = threadIdx.x;
  for (int d = lane; d < D; d += 64) xr[d] = f2bf(s_row[d]);
}

// apply_rope over [S, H, D] rows of q (heads [0, Hq)) and k (heads
// [Hq, Hq+Hkv)), the token of cache row start_pos + s: one wave per
// (head, token).
template <int D>
__global__ __launch_bounds__(64) void rope_kernel(bf16* __restrict__ q, bf16* __restrict__ k, int Hq, int Hkv,
                                                 int start_pos, int rot, RopeFreq rf, RopePos ropep) {
  __shared__ float s_row[D];
  const int s = blockIdx.x, hh = blockIdx.y;   // tokens on x: no 65535 cap on S
  bf16* row = hh < Hq ? q + (static_cast<size_t>(s) * Hq + hh) * D : k + (static_cast<size_t>(s) * Hkv + hh - Hq) * D;
  const int lane = threadIdx.x;
  for (int d = lane; d < D; d += 64) s_row[d] = bf2f(row[d]);
  __syncthreads();
  rope_from_lds<D>(s_row, row, rot, rope_row_pos(ropep, 0, start_pos + s), ropep, rf);
}

// o = in * sigmoid(g), 8 elements per thread where n allows.
__global__ void sigmoid_mul_kernel(const bf16* __restrict__ in, const bf16* __restrict__ g, bf16* __restrict__ o,
                                   long n) {
  const long n8 = n / 8;
  for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < n8;
       i += static_cast<long>(gridDim.x) * blockDim.x) {
    float a[8], gg[8];
    unpack8(ld16(in + i * 8), a);
    unpack8(ld16(g + i * 8), gg);
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x0 = a[2 * e] * (1.0f / (1.0f + expf(-gg[2 * e])));
      const float x1 = a[2 * e + 1] * (1.0f / (1.0f + expf(-gg[2 * e + 1])));
      w[e] = static_cast<uint32_t>(f2bf(x0)) | (static_cast<uint32_t>(f2bf(x1)) << 16);
    }
    *reinterpret_cast<u32x4*>(o + i * 8) = w;
  }
  // tail (n % 8) by the first threads
  const long t = n8 * 8 + blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x;
  if (t < n && blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x < 8)
    o[t] = f2bf(bf2f(in[t]) * (1.0f / (1.0f + expf(-bf2f(g[t])))));
}

int clamp_rot(int D, int rotary_dim) {
  int rot = std::max(2, std::min(D, rotary_dim));
  if (rot & 1) --rot;
  return rot;
}

template <typename F>
int with_d(int D, const char* what, F&& f) {
  switch (D) {
    case 64: return f(std::integral_constant<int, 64>{});
    case 128: return f(std::integral_constant<int, 128>{});
    case 256: return f(std::integral_constant<int, 256>{});
    default: return set_error(AILA_HIP_EUNSUPPORTED, "%s: D=%d not in {64,128,256}", what, D);
  }
}

}  // namespace
}  // namespace aila

extern "C" int aila_hip_decode_prepare_qkv(const void* q_in, int packed_gate, void* q_out, void* gate_out,
                                           void* k, const void* v, const void* q_norm_w, const void* k_norm_w,
                                           void* k_cache, void* v_cache, int B, int Hq, int Hkv, int D,
                                           int max_seq, int rotary_dim, float theta, float eps, int pos,
                                           const int* positions, const aila_hip_rope_pos* rope_pos,
                                           void* stream) {
  using namespace aila;
  RopePos rpd;
  if (int rc = load_rope_pos(rope_pos, &rpd, "decode_prepare_qkv")) return rc;
  AILA_REQUIRE(q_in && q_out && k && v, "decode_prepare_qkv: null pointer");
  AILA_REQUIRE(B > 0 && B <= 65535 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0,
               "decode_prepare_qkv: bad shape (B=%d Hq=%d Hkv=%d)", B, Hq, Hkv);
  AILA_REQUIRE(!packed_gate || gate_out, "decode_prepare_qkv: packed input needs gate_out");
  AILA_REQUIRE((k_cache == nullptr) == (v_cache == nullptr), "decode_prepare_qkv: pass both caches or neither");
  AILA_REQUIRE(!k_cache || max_seq > 0, "decode_prepare_qkv: max_seq=%d", max_seq);
  AILA_REQUIRE(!k_cache || positions || (pos >= 0 && pos < max_seq),
               "decode_prepare_qkv: pos=%d outside [0, max_seq=%d)", pos, max_seq);
  AILA_REQUIRE(theta > 0.f && eps >= 0.f, "decode_prepare_qkv: theta=%g eps=%g", theta, eps);
  const int rot = clamp_rot(D, rotary_dim);
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_d(D, "decode_prepare_qkv", [&](auto dc) {
    constexpr int DD = decltype(dc)::value;
    hipLaunchKernelGGL((decode_prep_kernel<DD>), dim3(Hq + Hkv, B), dim3(64), 0, st,
                       static_cast<const bf16*>(q_in), packed_gate ? 2 * DD : DD, static_cast<bf16*>(q_out),
                       packed_gate ? static_cast<bf16*>(gate_out) : nullptr, static_cast<bf16*>(k),
                       static_cast<const bf16*>(v), static_cast<const bf16*>(q_norm_w),
                       static_cast<const bf16*>(k_norm_w), static_cast<bf16*>(k_cache),
                       static_cast<bf16*>(v_cache), Hq, Hkv, max_seq, rot, rope_freq_table(theta, rot), eps, pos,
                       positions, rpd);
    return check_launch("decode_prepare_qkv");
  });
}

extern "C" int aila_hip_head_rms_norm(void* x, const void* weight, int S, int H, int D, float eps, void* stream) {
  using namespace aila;
  AILA_REQUIRE(x, "head_rms_norm: null pointer");
  AILA_REQUIRE(S >= 0 && H > 0 && eps >= 0.f, "head_rms_norm: bad shape (S=%d H=%d)", S, H);
  const long rows = static_cast<long>(S) * H;
  if (rows == 0) return AILA_HIP_OK;
  const unsigned gx = static_cast<unsigned>(std::min<long>(rows, 65535));
  const unsigned gy = static_cast<unsigned>((rows + gx - 1) / gx);
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_d(D, "head_rms_norm", [&](auto dc) {
    constexpr int DD = decltype(dc)::value;
    hipLaunchKernelGGL((head_rms_norm_kernel<DD>), dim3(gx, gy), dim3(64), 0, st, static_cast<bf16*>(x),
                       static_cast<const bf16*>(weight), eps, rows);
    return check_launch("head_rms_norm");
  });
}

extern "C" int aila_hip_apply_rope(void* q, void* k, int S, int start_pos, int Hq, int Hkv, int D, int rotary_dim,
                                   float theta, const aila_hip_rope_pos* rope_pos, void* stream) {
  using namespace aila;
  AILA_REQUIRE(q && k, "apply_rope: null pointer");
  RopePos rpd;
  if (int rc = load_rope_pos(rope_pos, &rpd, "apply_rope")) return rc;
  AILA_REQUIRE(S >= 0 && start_pos >= 0 && Hq > 0 && Hkv > 0 && Hkv <= Hq && Hq + Hkv <= 65535 && theta > 0.f,
               "apply_rope: bad shape (S=%d start_pos=%d Hq=%d Hkv=%d)", S, start_pos, Hq, Hkv);
  if (S == 0) return AILA_HIP_OK;
  const int rot = clamp_rot(D, rotary_dim);
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_d(D, "apply_rope", [&](auto dc) {
    constexpr int DD = decltype(dc)::value;
    hipLaunchKernelGGL((rope_kernel<DD>), dim3(S, Hq + Hkv), dim3(64), 0, st, static_cast<bf16*>(q),
                       static_cast<bf16*>(k), Hq, Hkv, start_pos, rot, rope_freq_table(theta, rot), rpd);
    return check_launch("apply_rope");
  });
}

extern "C" int aila_hip_sigmoid_mul(const void* input, const void* gate, void* output, long n, void* stream) {
  using namespace aila;
  AILA_REQUIRE(input && gate && output, "sigmoid_mul: null pointer");
  AILA_REQUIRE(n >= 0, "sigmoid_mul: n=%ld", n);
  if (n == 0) return AILA_HIP_OK;
  const long n8 = std::max<long>(1, n / 8);
  const int blocks = static_cast<int>(std::min<long>((n8 + 255) / 256, 8192));
  hipLaunchKernelGGL(sigmoid_mul_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const bf16*>(input), static_cast<const bf16*>(gate), static_cast<bf16*>(output), n);
  return check_launch("sigmoid_mul");
}

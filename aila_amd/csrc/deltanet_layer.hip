// The whole Gated DeltaNet layer around the recurrence, one token per
// sequence: causal conv1d (kernel 4) over the packed [q | k | v] row with a
// ring of the three previous raw rows, SiLU, per-head L2 norm of q and k,
// the gated delta update of the fp32 state, o = scale * S^T q, and the
// output gate RMSNorm(o) * norm_w * SiLU(z).
//
// Reference: the fast path of Qwen35HybridTextBackend::run_linear_delta_decode_gpu
// (src/models/Qwen35HybridTextBackend.cpp:1013-1166; ring rows head, head+1,
// head+2 weighted by w[0..2], the new row by w[3], then written to row head),
// host form run_linear_delta_host (:1640-1798), output gate :153-173.
//
// Work decomposition: one workgroup of 256*G threads per (key head,
// sequence), G = Hv / Hk value heads sharing that key head. The workgroup
// is the only reader and writer of its conv channels (q and k of the key
// head, v of its G value heads), so the ring row it reads as oldest can be
// overwritten in the same launch without a race between workgroups (the
// reference's per-value-head launch lets the group leader overwrite the
// shared q/k ring row while the other value heads of the group may still
// read it). Within a value head the state slab is held in VGPRs between the
// two reductions, as in the recurrence-only decode kernel: 1 read + 1 write
// of the state per step.
#include "common.hpp"

namespace aila {
namespace {

constexpr int kD = 128;          // dk = dv = 128 (the reference fast path's shape)
constexpr int kConvK = 4;        // conv kernel width (ring of 3 rows)
constexpr int kRows = kConvK - 1;
constexpr int kColQuads = 32;
constexpr int kRowGroups = 8;
constexpr int kRPT = kD / kRowGroups;

template <int G>
__global__ __launch_bounds__(256 * G) void deltanet_layer_decode_kernel(
    const bf16* __restrict__ qkv, int qkv_stride, const bf16* __restrict__ z, int z_stride,
    const bf16* __restrict__ a, const bf16* __restrict__ bgate, int ab_stride,
    const bf16* __restrict__ conv_w, float* __restrict__ conv_state, int conv_head,
    const int* __restrict__ conv_heads, const bf16* __restrict__ dt_bias, const float* __restrict__ A_log,
    const float* __restrict__ norm_w, float* __restrict__ state, bf16* __restrict__ out, int Hk, float eps,
    float scale) {
  const int hk = blockIdx.x, bseq = blockIdx.y;
  const int Hv = Hk * G;
  const int qd = Hk * kD, ch = 2 * qd + Hv * kD;
  const int t = threadIdx.x;
  const int g = t >> 8, tt = t & 255;
  const int cq = tt % kColQuads, rg = tt / kColQuads;
  const int col = cq * 4;
  const int hv = hk * G + g;
  const int lane = t & 63, wave_in_head = tt >> 6;

  __shared__ float s_act[(2 + G) * kD];         // conv+SiLU outputs: q, k, v of G heads
  __shared__ float s_red[G][2][4][kColQuads * 4];

  float* S = state + (static_cast<size_t>(bseq) * Hv + hv) * kD * kD;

  // 1. Convolution inputs and gate scalars first, then the state slab: the
  //    convolution waits only for its own loads (in-order vmcnt) while the
  //    state loads stay in flight. Each channel's ring entries are read and
  //    then overwritten by one thread.
  constexpr int kCh = (2 + G) * kD;
  constexpr int kCPT = (kCh + 256 * G - 1) / (256 * G);   // channels per thread
  int head = conv_heads ? conv_heads[bseq] : conv_head;
  head = ((head % kRows) + kRows) % kRows;
  const int head1 = head == kRows - 1 ? 0 : head + 1;
  const int head2 = head == 0 ? kRows - 1 : head - 1;     // (head + 2) % 3
  const bf16* x = qkv + static_cast<size_t>(bseq) * qkv_stride;
  float* ring = conv_state + static_cast<size_t>(bseq) * kRows * ch;
  int cidx[kCPT];
  uint2 wr[kCPT];
  float xv[kCPT], h0[kCPT], h1[kCPT], h2[kCPT];
#pragma unroll
  for (int i = 0; i < kCPT; ++i) {
    const int lc = t + i * 256 * G;
    const int lcc = lc < kCh ? lc : kCh - 1;     // clamped: loads stay unconditional
    const int c = lcc < kD ? hk * kD + lcc
                           : (lcc < 2 * kD ? qd + hk * kD + lcc - kD : 2 * qd + hk * G * kD + lcc - 2 * kD);
    cidx[i] = c;
    wr[i] = *reinterpret_cast<const uint2*>(conv_w + static_cast<size_t>(c) * kConvK);
    xv[i] = bf2f(x[c]);
    h0[i] = ring[static_cast<size_t>(head) * ch + c];
    h1[i] = ring[static_cast<size_t>(head1) * ch + c];
    h2[i] = ring[static_cast<size_t>(head2) * ch + c];
  }
  const size_t ai = static_cast<size_t>(bseq) * ab_stride + hv;
  const float b_raw = bf2f(bgate[ai]);
  const float a_raw = bf2f(a[ai]);
  const float dtb = dt_bias ? bf2f(dt_bias[hv]) : 0.0f;
  const float alog = A_log ? A_log[hv] : 0.0f;
  const f32x4 nw = *reinterpret_cast<const f32x4*>(norm_w + col);
  const uint2 zr = *reinterpret_cast<const uint2*>(z + static_cast<size_t>(bseq) * z_stride + hv * kD + col);

  f32x4 s[kRPT];
#pragma unroll
  for (int r = 0; r < kRPT; ++r)
    s[r] = *reinterpret_cast<const f32x4*>(S + static_cast<size_t>(rg * kRPT + r) * kD + col);

  // 2. Convolution + SiLU into LDS; the new raw row replaces the oldest.
#pragma unroll
  for (int i = 0; i < kCPT; ++i) {
    const int lc = t + i * 256 * G;
    if (lc < kCh) {
      float acc = h0[i] * __uint_as_float(wr[i].x << 16);
      acc += h1[i] * __uint_as_float(wr[i].x & 0xffff0000u);
      acc += h2[i] * __uint_as_float(wr[i].y << 16);
      acc += xv[i] * __uint_as_float(wr[i].y & 0xffff0000u);
      s_act[lc] = silu_f(acc);
      ring[static_cast<size_t>(head) * ch + cidx[i]] = xv[i];
    }
  }

  // Gates (uniform per value head).
  const float beta = 1.0f / (1.0f + expf(-b_raw));
  const float negA = A_log ? -expf(alog) : -1.0f;
  const float decay = expf(softplus_f(a_raw + dtb) * negA);
  __syncthreads();

  // 3. L2 norms of q and k (every wave reduces both 128-vectors itself).
  float sq = s_act[lane] * s_act[lane] + s_act[lane + 64] * s_act[lane + 64];
  float sk = s_act[kD + lane] * s_act[kD + lane] + s_act[kD + lane + 64] * s_act[kD + lane + 64];
  sq = wave_sum(sq);
  sk = wave_sum(sk);
  const float qn = 1.0f / sqrtf(sq + eps);
  const float kn = 1.0f / sqrtf(sk + eps);

  // 4. S *= decay; u = S^T k (this thread's rows).
  float kr[kRPT];
  f32x4 u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < kRPT; ++r) {
    kr[r] = s_act[kD + rg * kRPT + r] * kn;
    s[r] *= decay;
    u += s[r] * kr[r];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) u[e] += __shfl_xor(u[e], 32);
  if (lane < 32) *reinterpret_cast<f32x4*>(&s_red[g][0][wave_in_head][cq * 4]) = u;
  __syncthreads();
  u = *reinterpret_cast<const f32x4*>(&s_red[g][0][0][cq * 4]) +
      *reinterpret_cast<const f32x4*>(&s_red[g][0][1][cq * 4]) +
      *reinterpret_cast<const f32x4*>(&s_red[g][0][2][cq * 4]) +
      *reinterpret_cast<const f32x4*>(&s_red[g][0][3][cq * 4]);

  // 5. d = (v - u) beta; S += k d^T; o = S^T q; one write of the state.
  const f32x4 vv = *reinterpret_cast<const f32x4*>(&s_act[(2 + g) * kD + col]);
  const f32x4 d = (vv - u) * beta;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < kRPT; ++r) {
    const float qr = s_act[rg * kRPT + r] * qn;
    s[r] += kr[r] * d;
    o += s[r] * qr;
  }
#pragma unroll
  for (int r = 0; r < kRPT; ++r)
    *reinterpret_cast<f32x4*>(S + static_cast<size_t>(rg * kRPT + r) * kD + col) = s[r];
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] += __shfl_xor(o[e], 32);
  if (lane < 32) *reinterpret_cast<f32x4*>(&s_red[g][1][wave_in_head][cq * 4]) = o;
  __syncthreads();

  // 6. Output gate on lanes 0..31 of the head's first wave (4 columns each):
  //    RMSNorm over the 128 outputs, * norm_w * SiLU(z), rounded to bf16.
  if (tt < kColQuads) {
    o = *reinterpret_cast<const f32x4*>(&s_red[g][1][0][cq * 4]) +
        *reinterpret_cast<const f32x4*>(&s_red[g][1][1][cq * 4]) +
        *reinterpret_cast<const f32x4*>(&s_red[g][1][2][cq * 4]) +
        *reinterpret_cast<const f32x4*>(&s_red[g][1][3][cq * 4]);
    o *= scale;
    float ss = o[0] * o[0] + o[1] * o[1] + o[2] * o[2] + o[3] * o[3];
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(kD) + eps);
    const float zf[4] = {__uint_as_float(zr.x << 16), __uint_as_float(zr.x & 0xffff0000u),
                         __uint_as_float(zr.y << 16), __uint_as_float(zr.y & 0xffff0000u)};
    float r4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) r4[e] = o[e] * inv * nw[e] * silu_f(zf[e]);
    uint2 w;
    w.x = pack_bf16x2(r4[0], r4[1]);
    w.y = pack_bf16x2(r4[2], r4[3]);
    *reinterpret_cast<uint2*>(out + (static_cast<size_t>(bseq) * Hv + hv) * kD + col) = w;
  }
}

bool aligned(const void* p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

}  // namespace
}  // namespace aila

extern "C" int aila_hip_deltanet_layer_decode(const void* qkv, int qkv_stride, const void* z, int z_stride,
                                              const void* a, const void* b, int ab_stride, const void* conv_w,
                                              float* conv_state, int conv_head, const int* conv_heads,
                                              const void* dt_bias, const float* A_log, const float* norm_w,
                                              float* state, void* out, int B, int Hk, int Hv, int dk, int dv,
                                              int conv_kernel, float eps, float scale, void* stream) {
  using namespace aila;
  AILA_REQUIRE(qkv && z && a && b && conv_w && conv_state && norm_w && state && out,
               "deltanet_layer_decode: null pointer");
  AILA_REQUIRE(dk == kD && dv == kD && conv_kernel == kConvK,
               "deltanet_layer_decode: needs dk = dv = 128 and conv kernel 4 (dk=%d dv=%d K=%d)", dk, dv,
               conv_kernel);
  AILA_REQUIRE(B > 0 && B <= 65535 && Hk > 0 && Hv > 0 && Hv % Hk == 0,
               "deltanet_layer_decode: bad B/Hk/Hv (B=%d Hk=%d Hv=%d)", B, Hk, Hv);
  const int ch = 2 * Hk * dk + Hv * dv;
  AILA_REQUIRE(qkv_stride >= ch && z_stride >= Hv * dv && ab_stride >= Hv,
               "deltanet_layer_decode: row strides too small (qkv %d < %d, z %d, ab %d)", qkv_stride, ch,
               z_stride, ab_stride);
  AILA_REQUIRE(aligned(conv_w, 8) && aligned(z, 8) && z_stride % 4 == 0 && aligned(norm_w, 16) &&
                   aligned(state, 16) && aligned(out, 8),
               "deltanet_layer_decode: misaligned conv_w/z/norm_w/state/out");
  const int G = Hv / Hk;
  const dim3 grid(Hk, B);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto* qp = static_cast<const bf16*>(qkv);
  auto* zp = static_cast<const bf16*>(z);
  auto* ap = static_cast<const bf16*>(a);
  auto* bp = static_cast<const bf16*>(b);
  auto* wp = static_cast<const bf16*>(conv_w);
  auto* dtp = static_cast<const bf16*>(dt_bias);
  auto* op = static_cast<bf16*>(out);
#define AILA_LAYER_DECODE(GG)                                                                              \
  hipLaunchKernelGGL(deltanet_layer_decode_kernel<GG>, grid, dim3(256 * GG), 0, st, qp, qkv_stride, zp,    \
                     z_stride, ap, bp, ab_stride, wp, conv_state, conv_head, conv_heads, dtp, A_log, norm_w, \
                     state, op, Hk, eps, scale)
  switch (G) {
    case 1: AILA_LAYER_DECODE(1); break;
    case 2: AILA_LAYER_DECODE(2); break;
    case 4: AILA_LAYER_DECODE(4); break;
    default:
      return set_error(AILA_HIP_EUNSUPPORTED, "deltanet_layer_decode: Hv/Hk = %d not in {1,2,4}", G);
  }
#undef AILA_LAYER_DECODE
  return check_launch("deltanet_layer_decode");
}

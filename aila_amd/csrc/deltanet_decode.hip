// Gated DeltaNet decode step on gfx950: a memory-bound rank-1 state update
// that reads and writes the fp32 state exactly once.
//
// Reference: Qwen35HybridTextBackend::run_linear_delta_decode_gpu
// (src/models/Qwen35HybridTextBackend.cpp:1013-1166) touches the state
// twice (a decay pass and an update pass, 2 reads + 2 writes). Here the
// state column slab lives in VGPRs between the two reductions.
//
// Work decomposition: one 256-thread workgroup per (value head, sequence,
// slab of 4*CQ columns of dv), CQ = 32, 16 or 8. Thread t owns columns
// 4*(t%CQ)..+3 of the slab and rows (t/CQ)*RPT..+RPT-1 of dk (RPT = dk /
// (256/CQ)). Loads are float4 along dv, so a wave reads 512- or 256-byte row
// segments per instruction. The column sums u = S^T k and o = S^T q are
// reduced over the row groups of a wave with lane swaps and over the 4
// waves through LDS. The narrower slabs (CQ = 16, 8) multiply the workgroups
// for small batches, where one workgroup per CU leaves the state load latency
// exposed (Hv = 32, dk = dv = 128, B = 8: 7.14 -> 6.70 us).
// State loads and stores are nontemporal: each step touches the state once
// and the next touch of the same state comes after every other layer's
// traffic. Measured with the state evicted from the caches (states used in
// rotation): B = 32, H = 16: 13.9 -> 12.1 us; B = 8, Hv = 32: 10.1 -> 7.2 us.
#include "common.hpp"
#include "deltanet_generic.hpp"

#include <type_traits>

namespace aila {
namespace {

constexpr int kThreads = 256;

template <int DK, int CQ>
__global__ __launch_bounds__(kThreads) void deltanet_decode_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k,
    const bf16* __restrict__ v, const bf16* __restrict__ a,
    const bf16* __restrict__ bgate, const bf16* __restrict__ dt_bias,
    const float* __restrict__ A_log, float* __restrict__ state,
    bf16* __restrict__ out, int Hk, int Hv, int dv, float eps, float scale) {
  constexpr int kColQuads = CQ;
  constexpr int kRowGroups = kThreads / CQ;
  constexpr int RPT = DK / kRowGroups;  // rows per thread
  const int hv = blockIdx.x;
  const int bseq = blockIdx.y;
  const int slab = blockIdx.z;
  const int t = threadIdx.x;
  const int cq = t % kColQuads;
  const int rg = t / kColQuads;
  const int col = slab * (kColQuads * 4) + cq * 4;
  const bool active = col < dv;          // dv % 4 == 0 is required
  const int hk = hv / (Hv / Hk);

  __shared__ float s_q[DK];
  __shared__ float s_k[DK];
  __shared__ float s_red[2][4][kColQuads * 4];
  __shared__ float s_norm[2][4];

  float* S = state + (static_cast<size_t>(bseq) * Hv + hv) * DK * dv;

  // 1. The small operands (q, k, v, gates) first, then the state slab: the
  //    norms wait only for their own loads (in-order vmcnt) while the state
  //    loads stay in flight, and v is in registers before the update.
  const bf16* qh = q + (static_cast<size_t>(bseq) * Hk + hk) * DK;
  const bf16* kh = k + (static_cast<size_t>(bseq) * Hk + hk) * DK;
  constexpr int kQK = (DK + kThreads - 1) / kThreads;
  float qf[kQK], kf[kQK];
#pragma unroll
  for (int j = 0; j < kQK; ++j) {
    const int i = t + j * kThreads < DK ? t + j * kThreads : DK - 1;
    qf[j] = bf2f(qh[i]);
    kf[j] = bf2f(kh[i]);
  }
  const size_t gi = static_cast<size_t>(bseq) * Hv + hv;
  const float b_raw = bf2f(bgate[gi]);
  const float a_raw = bf2f(a[gi]);
  const float dtb = dt_bias ? bf2f(dt_bias[hv]) : 0.0f;
  const float alog = A_log ? A_log[hv] : 0.0f;
  const uint2 vraw = *reinterpret_cast<const uint2*>(v + gi * dv + (active ? col : 0));

  f32x4 s[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int row = rg * RPT + r;
    s[r] = active ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(S + static_cast<size_t>(row) * dv + col))
                  : f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // 2. q, k L2 norms (head_l2_norm_inplace, :138-151 / :1079-1089).
  float sq = 0.f, sk = 0.f;
#pragma unroll
  for (int j = 0; j < kQK; ++j) {
    if (t + j * kThreads < DK) {
      s_q[t + j * kThreads] = qf[j];
      s_k[t + j * kThreads] = kf[j];
      sq += qf[j] * qf[j];
      sk += kf[j] * kf[j];
    }
  }
  sq = wave_sum(sq);
  sk = wave_sum(sk);
  const int wave = t >> 6, lane = t & 63;
  if (lane == 0) {
    s_norm[0][wave] = sq;
    s_norm[1][wave] = sk;
  }
  // Gates (Qwen35HybridTextBackend.cpp:1091-1099), uniform per head.
  const float beta = 1.0f / (1.0f + expf(-b_raw));
  const float negA = A_log ? -expf(alog) : -1.0f;
  const float decay = expf(softplus_f(a_raw + dtb) * negA);
  __syncthreads();
  const float qn = 1.0f / sqrtf(s_norm[0][0] + s_norm[0][1] + s_norm[0][2] + s_norm[0][3] + eps);
  const float kn = 1.0f / sqrtf(s_norm[1][0] + s_norm[1][1] + s_norm[1][2] + s_norm[1][3] + eps);

  // 3. S *= decay; partial u = S^T k over this thread's rows.
  float kr[RPT];
  f32x4 u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    kr[r] = s_k[rg * RPT + r] * kn;
    s[r] *= decay;
    u += s[r] * kr[r];
  }
  // The 64 / CQ row groups of wave w live in lane blocks of CQ.
#pragma unroll
  for (int m = CQ; m < 64; m <<= 1)
#pragma unroll
    for (int e = 0; e < 4; ++e) u[e] += __shfl_xor(u[e], m);
  if (lane < CQ) *reinterpret_cast<f32x4*>(&s_red[0][wave][cq * 4]) = u;
  __syncthreads();
  u = *reinterpret_cast<const f32x4*>(&s_red[0][0][cq * 4]) +
      *reinterpret_cast<const f32x4*>(&s_red[0][1][cq * 4]) +
      *reinterpret_cast<const f32x4*>(&s_red[0][2][cq * 4]) +
      *reinterpret_cast<const f32x4*>(&s_red[0][3][cq * 4]);

  // 4. d = (v - u) * beta ; S += k d^T ; partial o = S^T q.
  f32x4 vv;
  vv[0] = __uint_as_float(vraw.x << 16);
  vv[1] = __uint_as_float(vraw.x & 0xffff0000u);
  vv[2] = __uint_as_float(vraw.y << 16);
  vv[3] = __uint_as_float(vraw.y & 0xffff0000u);
  const f32x4 d = (vv - u) * beta;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const float qr = s_q[rg * RPT + r] * qn;
    s[r] += kr[r] * d;
    o += s[r] * qr;
  }
  // 5. Single write of the state.
  if (active) {
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const int row = rg * RPT + r;
      __builtin_nontemporal_store(s[r], reinterpret_cast<f32x4*>(S + static_cast<size_t>(row) * dv + col));
    }
  }
#pragma unroll
  for (int m = CQ; m < 64; m <<= 1)
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] += __shfl_xor(o[e], m);
  if (lane < CQ) *reinterpret_cast<f32x4*>(&s_red[1][wave][cq * 4]) = o;
  __syncthreads();
  if (t < kColQuads && active) {
    o = *reinterpret_cast<const f32x4*>(&s_red[1][0][cq * 4]) +
        *reinterpret_cast<const f32x4*>(&s_red[1][1][cq * 4]) +
        *reinterpret_cast<const f32x4*>(&s_red[1][2][cq * 4]) +
        *reinterpret_cast<const f32x4*>(&s_red[1][3][cq * 4]);
    o *= scale;
    uint2 w;
    w.x = pack_bf16x2(o[0], o[1]);
    w.y = pack_bf16x2(o[2], o[3]);
    *reinterpret_cast<uint2*>(out + gi * dv + col) = w;
  }
}

}  // namespace
}  // namespace aila

extern "C" int aila_hip_deltanet_decode(const void* q, const void* k,
                                        const void* v, const void* a,
                                        const void* b, const void* dt_bias,
                                        const float* A_log, float* state,
                                        void* out, int B, int Hk, int Hv,
                                        int dk, int dv, float eps, float scale,
                                        void* stream) {
  using namespace aila;
  AILA_REQUIRE(q && k && v && a && b && state && out, "deltanet_decode: null pointer");
  AILA_REQUIRE(B > 0 && Hk > 0 && Hv > 0 && dk > 0 && dv > 0,
               "deltanet_decode: need B, Hk, Hv, dk, dv > 0 (B=%d Hk=%d Hv=%d dk=%d dv=%d)", B, Hk, Hv, dk, dv);
  AILA_REQUIRE(B <= 65535, "deltanet_decode: B too large (%d)", B);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (Hv % Hk != 0 || dv % 4 != 0 || (dk != 64 && dk != 128 && dk != 256)) {
    // general shapes: one token of the sequential kernel
    GenericDeltaNet g{};
    g.q = static_cast<const bf16*>(q);
    g.k = static_cast<const bf16*>(k);
    g.v = static_cast<const bf16*>(v);
    g.a = static_cast<const bf16*>(a);
    g.b = static_cast<const bf16*>(b);
    g.ab_stride = Hv;
    g.dt_bias = static_cast<const bf16*>(dt_bias);
    g.A_log = A_log;
    g.state = state;
    g.out = static_cast<bf16*>(out);
    g.B = B, g.T = 1, g.Hk = Hk, g.Hv = Hv, g.dk = dk, g.dv = dv, g.K = 1;
    g.eps = eps, g.scale = scale;
    return deltanet_generic_launch(g, st, "deltanet_decode");
  }
  const bf16* qp = static_cast<const bf16*>(q);
  const bf16* kp = static_cast<const bf16*>(k);
  const bf16* vp = static_cast<const bf16*>(v);
  const bf16* ap = static_cast<const bf16*>(a);
  const bf16* bp = static_cast<const bf16*>(b);
  const bf16* dtp = static_cast<const bf16*>(dt_bias);
  bf16* op = static_cast<bf16*>(out);
  // 128-column slabs unless that leaves fewer than two workgroups per CU;
  // 32-column slabs when even 64-column ones leave CUs idle (batch 1-4 of
  // 32 value heads: B=1 4.1 -> 3.9 us, B=2 4.3 -> 4.15 us).
  const long heads = static_cast<long>(B) * Hv * ((dv + 127) / 128);
  const bool narrow = heads < 512;
  const bool narrower = heads <= 128;
  auto launch = [&](auto dk_tag, auto cq_tag) {
    constexpr int DK = decltype(dk_tag)::value, CQ = decltype(cq_tag)::value;
    const dim3 grid(Hv, B, (dv + CQ * 4 - 1) / (CQ * 4));
    hipLaunchKernelGGL((deltanet_decode_kernel<DK, CQ>), grid, dim3(kThreads), 0, st, qp, kp, vp, ap, bp, dtp,
                       A_log, state, op, Hk, Hv, dv, eps, scale);
  };
  auto with_cq = [&](auto dk_tag) {
    if (narrower) launch(dk_tag, std::integral_constant<int, 8>{});
    else if (narrow) launch(dk_tag, std::integral_constant<int, 16>{});
    else launch(dk_tag, std::integral_constant<int, 32>{});
  };
  switch (dk) {
    case 64: with_cq(std::integral_constant<int, 64>{}); break;
    case 128: with_cq(std::integral_constant<int, 128>{}); break;
    case 256: with_cq(std::integral_constant<int, 256>{}); break;
    default:
      return set_error(AILA_HIP_EUNSUPPORTED, "deltanet_decode: dk=%d not in {64,128,256}", dk);
  }
  return check_launch("deltanet_decode");
}

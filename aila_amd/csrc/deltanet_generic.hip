// General-shape Gated DeltaNet: the recurrence and the whole layer for the
// shapes the tuned kernels do not compile (dk or dv other than their sizes,
// any conv kernel width, value/key head ratios outside {1, 2, 4}, or a head
// count that does not divide). Role of the reference's single-workgroup
// fallback in Qwen35HybridTextBackend::run_linear_delta_decode_gpu
// (src/models/Qwen35HybridTextBackend.cpp:1168-1304) and of the token loop
// of run_linear_delta_prefill_gpu_batched (:1306-1508) for the same shapes.
//
// One 512-thread workgroup per (value head, sequence) walks the tokens in
// order. Lane l of wave w owns columns i = l + 64c (c < 4) and rows
// j = w + 8r, so dk, dv <= 256. The [dk x dv] fp32 state stays in global
// memory (at most 256 KiB per head, L2-resident across the walk): per token
// one pass forms u = (decay S)^T k, the second writes S <- decay S + k d^T
// and forms o = S^T q. This is the reference's own two-pass update
// (:1100-1142); the tuned kernels keep the state in registers instead, but a
// register tile sized for every shape up to 256 x 256 does not fit here.
// Per token: inputs (or, for the layer, the conv taps over the ring and the
// earlier tokens' raw rows, then SiLU) into LDS, the L2 norms of q and k, the
// two passes with their column sums over the 8 row groups through LDS, then
// o * scale (recurrence) or the gated RMSNorm (layer). The layer's conv ring
// is rewritten by a second launch, after every workgroup has read it.
#include "deltanet_generic.hpp"

#include <algorithm>

namespace aila {
namespace {

constexpr int kGWaves = 8;
constexpr int kGThreads = kGWaves * 64;
constexpr int kGCols = 4;    // 64-column groups per lane

// Key head of value head hv (Qwen35HybridTextBackend.cpp:104-118): contiguous
// groups when Hk divides Hv, else clamp(hv, 0, Hk - 1).
__device__ __forceinline__ int key_head_of(int hv, int Hk, int Hv) {
  if (Hv % Hk != 0) return min(max(hv, 0), Hk - 1);
  return min(hv / (Hv / Hk), Hk - 1);
}

__device__ __forceinline__ float block_sum(float x, float* s_part, int wave, int lane) {
  x = wave_sum(x);
  if (lane == 0) s_part[wave] = x;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kGWaves; ++w) t += s_part[w];
  return t;
}

__global__ __launch_bounds__(kGThreads) void deltanet_generic_kernel(GenericDeltaNet p) {
  __shared__ float s_q[256], s_k[256], s_v[256], s_z[256];
  __shared__ float s_red[kGWaves][256];
  __shared__ float s_vec[256];
  __shared__ float s_part[2][kGWaves];
  const int hv = blockIdx.x, bb = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int dk = p.dk, dv = p.dv;
  const int hk = key_head_of(hv, p.Hk, p.Hv);
  const int R = p.K - 1;
  int head = 0;
  if (p.layer && R > 0) {
    head = p.conv_heads ? p.conv_heads[bb] : p.conv_head;
    head = ((head % R) + R) % R;
  }
  const int ch = 2 * p.Hk * dk + p.Hv * dv;
  const float* ring = p.layer && R > 0 ? p.conv_state + static_cast<size_t>(bb) * R * ch : nullptr;

  float* Sg = p.state + (static_cast<size_t>(bb) * p.Hv + hv) * dk * dv;

  const float dtb = p.dt_bias ? bf2f(p.dt_bias[hv]) : 0.f;
  const float negA = p.A_log ? -expf(p.A_log[hv]) : -1.f;

  for (int t = 0; t < p.T; ++t) {
    const size_t bt = static_cast<size_t>(bb) * p.T + t;
    // ---- inputs: q, k of key head hk and v of value head hv, fp32 in LDS
    if (!p.layer) {
      for (int idx = tid; idx < dk; idx += kGThreads) {
        s_q[idx] = bf2f(p.q[(bt * p.Hk + hk) * dk + idx]);
        s_k[idx] = bf2f(p.k[(bt * p.Hk + hk) * dk + idx]);
      }
      for (int idx = tid; idx < dv; idx += kGThreads) s_v[idx] = bf2f(p.v[(bt * p.Hv + hv) * dv + idx]);
    } else {
      // conv taps: token t reads history entries n = t + jj (jj < R) of
      // [ring rows oldest first, token 0, token 1, ...], then its own row
      for (int idx = tid; idx < 2 * dk + dv; idx += kGThreads) {
        const int c = idx < dk ? hk * dk + idx
                               : idx < 2 * dk ? p.Hk * dk + hk * dk + (idx - dk) : 2 * p.Hk * dk + hv * dv + (idx - 2 * dk);
        const bf16* w = p.conv_w + static_cast<size_t>(c) * p.K;
        float acc = 0.f;
        for (int jj = 0; jj < R; ++jj) {
          const int n = t + jj;
          const float x = n < R ? ring[static_cast<size_t>((head + n) % R) * ch + c]
                                : bf2f(p.qkv[(static_cast<size_t>(bb) * p.T + (n - R)) * p.qkv_stride + c]);
          acc += x * bf2f(w[jj]);
        }
        acc += bf2f(p.qkv[bt * p.qkv_stride + c]) * bf2f(w[R]);
        const float y = silu_f(acc);
        if (idx < dk) s_q[idx] = y;
        else if (idx < 2 * dk) s_k[idx - dk] = y;
        else s_v[idx - 2 * dk] = y;
      }
      for (int idx = tid; idx < dv; idx += kGThreads)
        s_z[idx] = bf2f(p.z[bt * p.z_stride + static_cast<size_t>(hv) * dv + idx]);
    }
    __syncthreads();
    // ---- L2 norms of q and k (x / sqrt(sum x^2 + eps)) and the gates
    float sq = 0.f, sk = 0.f;
    for (int idx = tid; idx < dk; idx += kGThreads) {
      sq = fmaf(s_q[idx], s_q[idx], sq);
      sk = fmaf(s_k[idx], s_k[idx], sk);
    }
    sq = wave_sum(sq);
    sk = wave_sum(sk);
    if (lane == 0) {
      s_part[0][wave] = sq;
      s_part[1][wave] = sk;
    }
    __syncthreads();
    sq = 0.f;
    sk = 0.f;
#pragma unroll
    for (int w = 0; w < kGWaves; ++w) {
      sq += s_part[0][w];
      sk += s_part[1][w];
    }
    const float iq = 1.0f / sqrtf(sq + p.eps), ik = 1.0f / sqrtf(sk + p.eps);
    const float braw = bf2f(p.b[bt * p.ab_stride + hv]);
    const float araw = bf2f(p.a[bt * p.ab_stride + hv]);
    const float beta = 1.0f / (1.0f + expf(-braw));
    const float decay = expf(softplus_f(araw + dtb) * negA);
    // ---- u = (decay S)^T k
    float part[kGCols];
#pragma unroll
    for (int c = 0; c < kGCols; ++c) {
      const int i = c * 64 + lane;
      float u = 0.f;
      if (i < dv)
        for (int j = wave; j < dk; j += kGWaves) u = fmaf(Sg[static_cast<size_t>(j) * dv + i] * decay, s_k[j] * ik, u);
      part[c] = u;
    }
#pragma unroll
    for (int c = 0; c < kGCols; ++c)
      if (c * 64 + lane < dv) s_red[wave][c * 64 + lane] = part[c];
    __syncthreads();
    for (int i = tid; i < dv; i += kGThreads) {
      float u = 0.f;
#pragma unroll
      for (int w = 0; w < kGWaves; ++w) u += s_red[w][i];
      s_vec[i] = (s_v[i] - u) * beta;
    }
    __syncthreads();
    // ---- S <- decay S + k d^T; o = S^T q
#pragma unroll
    for (int c = 0; c < kGCols; ++c) {
      const int i = c * 64 + lane;
      float o = 0.f;
      if (i < dv) {
        const float di = s_vec[i];
        for (int j = wave; j < dk; j += kGWaves) {
          float* sp = Sg + static_cast<size_t>(j) * dv + i;
          const float sv = fmaf(s_k[j] * ik, di, *sp * decay);
          *sp = sv;
          o = fmaf(sv, s_q[j] * iq, o);
        }
      }
      part[c] = o;
    }
#pragma unroll
    for (int c = 0; c < kGCols; ++c)
      if (c * 64 + lane < dv) s_red[wave][c * 64 + lane] = part[c];
    __syncthreads();
    bf16* orow = p.out + bt * static_cast<size_t>(p.Hv) * dv + static_cast<size_t>(hv) * dv;
    float o = 0.f;
    if (tid < dv) {
#pragma unroll
      for (int w = 0; w < kGWaves; ++w) o += s_red[w][tid];
      o *= p.scale;
    }
    if (!p.layer) {
      if (tid < dv) orow[tid] = f2bf(o);
    } else {
      // gated RMSNorm over dv: o / sqrt(mean(o^2) + eps) * norm_w * silu(z)
      float ss = block_sum(tid < dv ? o * o : 0.f, s_part[0], wave, lane);
      const float rs = 1.0f / sqrtf(ss / static_cast<float>(dv) + p.eps);
      if (tid < dv) orow[tid] = f2bf(o * rs * p.norm_w[tid] * silu_f(s_z[tid]));
    }
    __syncthreads();   // LDS inputs and partials are rewritten by the next token
  }

}

// The conv ring after T tokens: slot s holds the raw row of the last token
// t with (head + t) % R == s (each token replaces the oldest row), or keeps
// its old row when no token reached it (T < R).
__global__ void deltanet_generic_ring_kernel(GenericDeltaNet p) {
  const int R = p.K - 1;
  const int ch = 2 * p.Hk * p.dk + p.Hv * p.dv;
  const int bb = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= ch) return;
  int head = p.conv_heads ? p.conv_heads[bb] : p.conv_head;
  head = ((head % R) + R) % R;
  float* ring = p.conv_state + static_cast<size_t>(bb) * R * ch;
  for (int s = 0; s < R; ++s) {
    const int t = p.T - 1 - (((head + p.T - 1 - s) % R) + R) % R;
    if (t >= 0) ring[static_cast<size_t>(s) * ch + c] = bf2f(p.qkv[(static_cast<size_t>(bb) * p.T + t) * p.qkv_stride + c]);
  }
}

}  // namespace

bool deltanet_generic_fits(int dk, int dv, int K) {
  return dk > 0 && dk <= 256 && dv > 0 && dv <= kGCols * 64 && K >= 1 && K <= 16;
}

int deltanet_generic_launch(const GenericDeltaNet& p, hipStream_t st, const char* what) {
  if (!deltanet_generic_fits(p.dk, p.dv, p.layer ? p.K : 1))
    return set_error(AILA_HIP_EUNSUPPORTED, "%s: dk=%d dv=%d conv kernel %d outside dk, dv <= 256, kernel <= 16",
                     what, p.dk, p.dv, p.K);
  if (p.B <= 0 || p.B > 65535 || p.Hk <= 0 || p.Hv <= 0 || p.T < 0)
    return set_error(AILA_HIP_EINVAL, "%s: bad shape (B=%d T=%d Hk=%d Hv=%d)", what, p.B, p.T, p.Hk, p.Hv);
  if (p.T == 0) return AILA_HIP_OK;
  hipLaunchKernelGGL(deltanet_generic_kernel, dim3(p.Hv, p.B), dim3(kGThreads), 0, st, p);
  if (p.layer && p.K > 1) {
    const int ch = 2 * p.Hk * p.dk + p.Hv * p.dv;
    hipLaunchKernelGGL(deltanet_generic_ring_kernel, dim3((ch + 255) / 256, p.B), dim3(256), 0, st, p);
  }
  return check_launch(what);
}

}  // namespace aila

// Ceiling probes for the benchmark: the HBM read rate this chip reaches
// over the GQA decode's exact K/V layout, the in-place read + write rate over
// a DeltaNet state, and the dense bf16 MFMA rate it sustains, reported beside the decode's and the prefill's rooflines as the
// achievable ceilings. Measurement only: they are built into their own
// library (libaila_probe.so), which the benchmark loads and the product
// never does.
//
// Streaming read:
// Grid (split, kv head, sequence), 256 threads, as the decode's split
// kernel: workgroup (s, h, b) reads rows [s*len/nsplit, (s+1)*len/nsplit)
// of K[b, h] and of V[b, h] (cache [B, Hkv, max_seq, D] bf16) once, with
// 16-byte nontemporal loads, sixteen in flight per thread, and folds them
// into a value that is stored only if it equals a constant no input
// produces in practice (so the loads cannot be dropped).
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int kThreads = 256;
constexpr int kUnroll = 16;

__global__ __launch_bounds__(kThreads) void stream_read_kernel(const unsigned char* __restrict__ k,
                                                               const unsigned char* __restrict__ v, int Hkv,
                                                               long max_seq, long len, int D, unsigned* sink) {
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const long rows = (len + gridDim.x - 1) / gridDim.x;
  const long r0 = split * rows, r1 = r0 + rows < len ? r0 + rows : len;
  if (r0 >= r1) return;
  const size_t row_bytes = static_cast<size_t>(D) * 2;
  const size_t base = ((static_cast<size_t>(b) * Hkv + h) * max_seq + r0) * row_bytes;
  const size_t n16 = (r1 - r0) * row_bytes / 16;
  uint32_t acc = 0;
  for (int t = 0; t < 2; ++t) {
    const u32x4* p = reinterpret_cast<const u32x4*>((t == 0 ? k : v) + base);
    size_t i = threadIdx.x;
    for (; i + (kUnroll - 1) * kThreads < n16; i += kUnroll * kThreads) {
      u32x4 x[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) x[u] = __builtin_nontemporal_load(p + i + u * kThreads);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) acc ^= x[u][0] ^ x[u][1] ^ x[u][2] ^ x[u][3];
    }
    for (; i < n16; i += kThreads) {
      const u32x4 x = __builtin_nontemporal_load(p + i);
      acc ^= x[0] ^ x[1] ^ x[2] ^ x[3];
    }
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

// In-place read + write: every 16-byte chunk of a buffer is read and
// written back (nontemporal both ways, sixteen in flight per thread), the
// traffic of a DeltaNet decode step over its fp32 state with no
// arithmetic. The value written is the value read XOR `key`, a kernel
// argument the host passes as 0: the buffer keeps its contents, and the
// compiler cannot drop the store (or with it the load) as a copy of a
// location onto itself.
__global__ __launch_bounds__(kThreads) void stream_rw_kernel(u32x4* __restrict__ p, size_t n16, unsigned key) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
    u32x4 x[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) x[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) __builtin_nontemporal_store(x[u] ^ key, p + i + u * stride);
  }
  for (; i < n16; i += stride) __builtin_nontemporal_store(__builtin_nontemporal_load(p + i) ^ key, p + i);
}

// Dense MFMA: every wave issues `iters` rounds of 16 independent
// v_mfma_f32_16x16x32_bf16 (16,384 FLOP each) on register operands; the
// accumulators are folded and stored only if they equal a constant no run
// produces, so nothing is dropped. Two waves per SIMD, as the prefill runs.
constexpr int kAcc = 16;
__global__ __launch_bounds__(kThreads) void mfma_kernel(int iters, float seed, float* sink) {
  const float x = seed + static_cast<float>(threadIdx.x & 7) * 0.001f;
  bf16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = static_cast<__bf16>(x + e * 0.01f);
    b[e] = static_cast<__bf16>(x - e * 0.01f);
  }
  f32x4 c[kAcc];
#pragma unroll
  for (int j = 0; j < kAcc; ++j) c[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kAcc; ++j) c[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c[j], 0, 0, 0);
  }
  float t = 0.f;
#pragma unroll
  for (int j = 0; j < kAcc; ++j) t += c[j][0] + c[j][1] + c[j][2] + c[j][3];
  if (t == 1234.5f) sink[0] = t;
}

}  // namespace

// Reads rows [0, len) of every (sequence, kv head) of k_cache and v_cache
// ([B, Hkv, max_seq, D] bf16) once, in nsplit workgroups per (sequence, kv
// head). sink: one device unsigned. Returns a hipError_t.
extern "C" int aila_probe_stream_read(const void* k_cache, const void* v_cache, int B, int Hkv, long max_seq,
                                      long len, int D, int nsplit, unsigned* sink, void* stream) {
  if (!k_cache || !v_cache || !sink || B <= 0 || B > 65535 || Hkv <= 0 || Hkv > 65535 || nsplit <= 0 ||
      len <= 0 || len > max_seq || D <= 0 || (D * 2) % 16 != 0)
    return static_cast<int>(hipErrorInvalidValue);
  hipLaunchKernelGGL(stream_read_kernel, dim3(nsplit, Hkv, B), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const unsigned char*>(k_cache),
                     static_cast<const unsigned char*>(v_cache), Hkv, max_seq, len, D, sink);
  return static_cast<int>(hipGetLastError());
}

// Reads and writes back `bytes` (a multiple of 16) of `buf` in place, with
// `blocks` workgroups of 256 threads. Returns a hipError_t.
extern "C" int aila_probe_stream_rw(void* buf, size_t bytes, int blocks, void* stream) {
  if (!buf || bytes % 16 != 0 || blocks <= 0 || reinterpret_cast<uintptr_t>(buf) % 16 != 0)
    return static_cast<int>(hipErrorInvalidValue);
  if (bytes == 0) return 0;
  hipLaunchKernelGGL(stream_rw_kernel, dim3(blocks), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<u32x4*>(buf), bytes / 16, 0u);
  return static_cast<int>(hipGetLastError());
}

// Runs `blocks` workgroups of 256 threads (four waves), each wave issuing
// iters * 16 dense 16x16x32 bf16 MFMAs; FLOPs = blocks * 4 * iters * 16 *
// 16384. sink: one device float. Returns a hipError_t.
extern "C" int aila_probe_mfma(int blocks, int iters, float* sink, void* stream) {
  if (!sink || blocks <= 0 || iters <= 0) return static_cast<int>(hipErrorInvalidValue);
  hipLaunchKernelGGL(mfma_kernel, dim3(blocks), dim3(kThreads), 0, static_cast<hipStream_t>(stream), iters, 0.5f,
                     sink);
  return static_cast<int>(hipGetLastError());
}

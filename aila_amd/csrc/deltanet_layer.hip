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
#include "deltanet_generic.hpp"

namespace aila {

// Chunked prefill of the recurrence (deltanet_prefill.hip).
size_t deltanet_chunk_records_bytes(int B, int T, int Hv, bool split);
// conv == nullptr: q, k, v planes; else the layer (q, k, v formed from conv->qkv).
void launch_deltanet_chunked(const bf16* q, const bf16* k, const bf16* v, const ConvIn* conv, const bf16* a,
                             const bf16* b, int ab_stride, const bf16* dt_bias, const float* A_log, float* state,
                             bf16* out, unsigned char* records, int B, int T, int Hk, int Hv, float eps, float scale,
                             hipStream_t st);

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
    s[r] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(S + static_cast<size_t>(rg * kRPT + r) * kD + col));

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
    __builtin_nontemporal_store(s[r], reinterpret_cast<f32x4*>(S + static_cast<size_t>(rg * kRPT + r) * kD + col));
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

// One workgroup of 256 threads per (value head, sequence): twice (G = 2) or
// four times (G = 4) the workgroups of the kernel above, for batches that
// leave CUs idle with one workgroup per key head. The G workgroups of a key
// head all read the q/k ring rows of that key head; the one that arrives
// last - after every other has finished reading them, counted with one
// device-scope atomic per (sequence, key head) in the caller's `arrivals`
// array - writes the new q/k raw row there and resets the count to zero.
// Each workgroup writes the ring entries of its own v channels.
template <int G, int NT>
__global__ __launch_bounds__(NT) void deltanet_layer_decode_vh_kernel(
    const bf16* __restrict__ qkv, int qkv_stride, const bf16* __restrict__ z, int z_stride,
    const bf16* __restrict__ a, const bf16* __restrict__ bgate, int ab_stride,
    const bf16* __restrict__ conv_w, float* __restrict__ conv_state, int conv_head,
    const int* __restrict__ conv_heads, const bf16* __restrict__ dt_bias, const float* __restrict__ A_log,
    const float* __restrict__ norm_w, float* __restrict__ state, bf16* __restrict__ out, int Hk, float eps,
    float scale, unsigned int* __restrict__ arrivals) {
  const int hv = blockIdx.x, bseq = blockIdx.y;
  const int hk = hv / G;
  const int Hv = Hk * G;
  const int qd = Hk * kD, ch = 2 * qd + Hv * kD;
  constexpr int NW = NT / 64;                   // waves
  constexpr int RPT = kD / (NT / kColQuads);    // state rows per thread
  const int t = threadIdx.x;
  const int cq = t % kColQuads, rg = t / kColQuads;
  const int col = cq * 4;
  const int lane = t & 63, wave = t >> 6;

  __shared__ float s_act[3 * kD];               // conv+SiLU outputs: q, k, v
  __shared__ float s_red[2][NW][kColQuads * 4];
  __shared__ int s_last;

  float* S = state + (static_cast<size_t>(bseq) * Hv + hv) * kD * kD;

  // 1. conv inputs of q, k (key head hk) and v (value head hv), gates, then
  //    the state slab (the convolution waits only for its own loads)
  constexpr int kCh = 3 * kD;
  constexpr int kCPT = (kCh + NT - 1) / NT;
  int head = conv_heads ? conv_heads[bseq] : conv_head;
  head = ((head % kRows) + kRows) % kRows;
  const int head1 = head == kRows - 1 ? 0 : head + 1;
  const int head2 = head == 0 ? kRows - 1 : head - 1;
  const bf16* x = qkv + static_cast<size_t>(bseq) * qkv_stride;
  float* ring = conv_state + static_cast<size_t>(bseq) * kRows * ch;
  int cidx[kCPT];
  uint2 wr[kCPT];
  float xv[kCPT], h0[kCPT], h1[kCPT], h2[kCPT];
#pragma unroll
  for (int i = 0; i < kCPT; ++i) {
    const int lc = t + i * NT;
    const int lcc = lc < kCh ? lc : kCh - 1;
    const int c = lcc < kD ? hk * kD + lcc : (lcc < 2 * kD ? qd + hk * kD + lcc - kD : 2 * qd + hv * kD + lcc - 2 * kD);
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

  f32x4 s[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r)
    s[r] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(S + static_cast<size_t>(rg * RPT + r) * kD + col));

  // 2. conv + SiLU into LDS; own v channels' ring entries replaced now
#pragma unroll
  for (int i = 0; i < kCPT; ++i) {
    const int lc = t + i * NT;
    if (lc < kCh) {
      float acc = h0[i] * __uint_as_float(wr[i].x << 16);
      acc += h1[i] * __uint_as_float(wr[i].x & 0xffff0000u);
      acc += h2[i] * __uint_as_float(wr[i].y << 16);
      acc += xv[i] * __uint_as_float(wr[i].y & 0xffff0000u);
      s_act[lc] = silu_f(acc);
      if (lc >= 2 * kD) ring[static_cast<size_t>(head) * ch + cidx[i]] = xv[i];
    }
  }
  const float beta = 1.0f / (1.0f + expf(-b_raw));
  const float negA = A_log ? -expf(alog) : -1.0f;
  const float decay = expf(softplus_f(a_raw + dtb) * negA);
  __syncthreads();
  // Count this workgroup's arrival for the key head. Ordering of the shared
  // q/k ring row (read here by every workgroup of the key head, overwritten
  // by the last one to arrive): every thread consumed its ring values in the
  // convolution above before the barrier, so all of this workgroup's ring
  // loads have returned their data before thread 0 issues the count; the
  // last arriver's overwrite is issued only after its count returns (it is
  // control-dependent on the returned value). The count is therefore relaxed.
  // An agent-scope release here would write back this XCD's L2 in every
  // workgroup: measured 20.5 against 9.3 us per config-5 layer step.
  unsigned int* cnt = arrivals + static_cast<size_t>(bseq) * Hk + hk;
  unsigned int arrived = 0;
  if (t == 0) arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // 3. L2 norms of q and k
  float sq = s_act[lane] * s_act[lane] + s_act[lane + 64] * s_act[lane + 64];
  float sk = s_act[kD + lane] * s_act[kD + lane] + s_act[kD + lane + 64] * s_act[kD + lane + 64];
  sq = wave_sum(sq);
  sk = wave_sum(sk);
  const float qn = 1.0f / sqrtf(sq + eps);
  const float kn = 1.0f / sqrtf(sk + eps);

  // 4. S *= decay; u = S^T k
  float kr[RPT];
  f32x4 u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    kr[r] = s_act[kD + rg * RPT + r] * kn;
    s[r] *= decay;
    u += s[r] * kr[r];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) u[e] += __shfl_xor(u[e], 32);
  if (lane < 32) *reinterpret_cast<f32x4*>(&s_red[0][wave][cq * 4]) = u;
  if (t == 0) {
    const bool last = arrived == static_cast<unsigned int>(G - 1);
    if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  u = *reinterpret_cast<const f32x4*>(&s_red[0][0][cq * 4]);
#pragma unroll
  for (int w = 1; w < NW; ++w) u += *reinterpret_cast<const f32x4*>(&s_red[0][w][cq * 4]);
  // the last of the key head's workgroups replaces the q/k ring row
  if (s_last) {
#pragma unroll
    for (int i = 0; i < kCPT; ++i) {
      const int lc = t + i * NT;
      if (lc < 2 * kD) ring[static_cast<size_t>(head) * ch + cidx[i]] = xv[i];
    }
  }

  // 5. d = (v - u) beta; S += k d^T; o = S^T q; one write of the state
  const f32x4 vv = *reinterpret_cast<const f32x4*>(&s_act[2 * kD + col]);
  const f32x4 d = (vv - u) * beta;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const float qr = s_act[rg * RPT + r] * qn;
    s[r] += kr[r] * d;
    o += s[r] * qr;
  }
#pragma unroll
  for (int r = 0; r < RPT; ++r)
    __builtin_nontemporal_store(s[r], reinterpret_cast<f32x4*>(S + static_cast<size_t>(rg * RPT + r) * kD + col));
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] += __shfl_xor(o[e], 32);
  if (lane < 32) *reinterpret_cast<f32x4*>(&s_red[1][wave][cq * 4]) = o;
  __syncthreads();

  // 6. output gate: RMSNorm over the 128 outputs * norm_w * SiLU(z)
  if (t < kColQuads) {
    o = *reinterpret_cast<const f32x4*>(&s_red[1][0][cq * 4]);
#pragma unroll
    for (int w = 1; w < NW; ++w) o += *reinterpret_cast<const f32x4*>(&s_red[1][w][cq * 4]);
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

// ---- prefill epilogue: out = RMSNorm(o) * norm_w * SiLU(z), in place ------
// A (token, value head) row of 128 outputs per 16 lanes (8 per lane, one
// 16-byte access each); kGateRows rows per 256-thread block. Blocks past
// gate_blocks write the conv ring after T tokens: raw rows T-3, T-2, T-1 at
// ring rows (head + T + j) % 3 (a row whose token would be before token 0
// keeps its value). The chunk prep reads the old ring (tokens before 0), so
// the ring is rewritten only after it.
constexpr int kGateRows = 16 * 2;
__global__ __launch_bounds__(256) void deltanet_gate_kernel(bf16* __restrict__ out, const bf16* __restrict__ z,
                                                            int z_stride, const float* __restrict__ norm_w,
                                                            long rows, int Hv, float eps, int gate_blocks,
                                                            const bf16* __restrict__ qkv, int qkv_stride,
                                                            float* __restrict__ ring, int head, int T, int ch,
                                                            int B) {
  if (static_cast<int>(blockIdx.x) >= gate_blocks) {
    const long i = static_cast<long>(blockIdx.x - gate_blocks) * 256 + threadIdx.x;   // over [B][3][ch]
    if (i >= static_cast<long>(B) * kRows * ch) return;
    const int c = static_cast<int>(i % ch), j = static_cast<int>((i / ch) % kRows);
    const int bb = static_cast<int>(i / (static_cast<long>(kRows) * ch));
    const int t = T - kRows + j;
    if (t >= 0)
      ring[(static_cast<size_t>(bb) * kRows + (head + T + j) % kRows) * ch + c] =
          bf2f(qkv[(static_cast<size_t>(bb) * T + t) * qkv_stride + c]);
    return;
  }
  const int sub = threadIdx.x & 15;
  const f32x4 nw0 = *reinterpret_cast<const f32x4*>(norm_w + sub * 8);
  const f32x4 nw1 = *reinterpret_cast<const f32x4*>(norm_w + sub * 8 + 4);
  const float nw[8] = {nw0[0], nw0[1], nw0[2], nw0[3], nw1[0], nw1[1], nw1[2], nw1[3]};
  u32x4 ov[2], zv[2];
  long rowv[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {   // both rows' loads first
    const long row = static_cast<long>(blockIdx.x) * kGateRows + k * 16 + (threadIdx.x >> 4);
    rowv[k] = row;
    const long rr = row < rows ? row : rows - 1;
    const long bt = rr / Hv;
    const int hv = static_cast<int>(rr % Hv);
    ov[k] = ld16(out + rr * kD + sub * 8);
    zv[k] = ld16(z + bt * z_stride + hv * kD + sub * 8);
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    float o[8], zf[8], r[8];
    unpack8(ov[k], o);
    unpack8(zv[k], zf);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(o[e], o[e], ss);
    ss = row16_sum(ss);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(kD) + eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = o[e] * inv * nw[e] * silu_f(zf[e]);
    if (rowv[k] < rows)
      *reinterpret_cast<u32x4*>(out + rowv[k] * kD + sub * 8) =
          u32x4{pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]), pack_bf16x2(r[4], r[5]), pack_bf16x2(r[6], r[7])};
  }
}

// The prefill workspace holds the chunk records only (the prep forms q, k,
// v from the fused rows itself).
size_t layer_ws_bytes(int B, int T, int Hv) { return deltanet_chunk_records_bytes(B, T, Hv, true); }

}  // namespace

}  // namespace aila

extern "C" size_t aila_hip_deltanet_layer_prefill_workspace_size(int B, int T, int Hk, int Hv, int dk, int dv) {
  // 0 also for the shapes that run the sequential general-shape kernel
  if (B <= 0 || T <= 0 || Hk <= 0 || Hv <= 0 || dk != aila::kD || dv != aila::kD || Hv % Hk != 0) return 0;
  return aila::layer_ws_bytes(B, T, Hv);
}

extern "C" int aila_hip_deltanet_layer_prefill(const void* qkv, int qkv_stride, const void* z, int z_stride,
                                               const void* a, const void* b, int ab_stride, const void* conv_w,
                                               float* conv_state, int conv_head, const void* dt_bias,
                                               const float* A_log, const float* norm_w, float* state, void* out,
                                               void* workspace, size_t workspace_bytes, int B, int T, int Hk,
                                               int Hv, int dk, int dv, int conv_kernel, float eps, float scale,
                                               void* stream) {
  using namespace aila;
  AILA_REQUIRE(qkv && z && a && b && conv_w && conv_state && norm_w && state && out,
               "deltanet_layer_prefill: null pointer");
  AILA_REQUIRE(B > 0 && B <= 65535 && T > 0 && Hk > 0 && Hv > 0 && Hv <= 65535 && dk > 0 && dv > 0 &&
                   conv_kernel >= 1,
               "deltanet_layer_prefill: bad shape (B=%d T=%d Hk=%d Hv=%d dk=%d dv=%d K=%d)", B, T, Hk, Hv, dk, dv,
               conv_kernel);
  const int qd = Hk * dk, vd = Hv * dv, ch = 2 * qd + vd;
  AILA_REQUIRE(qkv_stride >= ch && z_stride >= vd && ab_stride >= Hv,
               "deltanet_layer_prefill: row strides too small (qkv %d < %d, z %d, ab %d)", qkv_stride, ch, z_stride,
               ab_stride);
  if (!(dk == kD && dv == kD && conv_kernel == kConvK && Hv % Hk == 0)) {
    // general shapes: the token-sequential layer kernel (no workspace)
    GenericDeltaNet g{};
    g.layer = 1;
    g.qkv = static_cast<const bf16*>(qkv);
    g.qkv_stride = qkv_stride;
    g.z = static_cast<const bf16*>(z);
    g.z_stride = z_stride;
    g.conv_w = static_cast<const bf16*>(conv_w);
    g.conv_state = conv_state;
    g.conv_head = conv_head;
    g.K = conv_kernel;
    g.norm_w = norm_w;
    g.a = static_cast<const bf16*>(a);
    g.b = static_cast<const bf16*>(b);
    g.ab_stride = ab_stride;
    g.dt_bias = static_cast<const bf16*>(dt_bias);
    g.A_log = A_log;
    g.state = state;
    g.out = static_cast<bf16*>(out);
    g.B = B, g.T = T, g.Hk = Hk, g.Hv = Hv, g.dk = dk, g.dv = dv;
    g.eps = eps, g.scale = scale;
    return deltanet_generic_launch(g, static_cast<hipStream_t>(stream), "deltanet_layer_prefill");
  }
  AILA_REQUIRE(aligned(qkv, 8) && qkv_stride % 4 == 0 && aligned(conv_w, 16) && aligned(conv_state, 16) &&
                   aligned(z, 16) && z_stride % 8 == 0 && aligned(norm_w, 16) && aligned(state, 16) &&
                   aligned(out, 16),
               "deltanet_layer_prefill: misaligned qkv/conv_w/conv_state/z/norm_w/state/out or odd strides");
  const size_t need = layer_ws_bytes(B, T, Hv);
  if (!workspace || workspace_bytes < need)
    return set_error(AILA_HIP_EWORKSPACE, "deltanet_layer_prefill: workspace %zu < %zu bytes", workspace_bytes,
                     need);
  // A sequence's fused rows are read through one buffer resource, a 2 GiB
  // byte range. Longer inputs run per sequence in consecutive segments of
  // whole chunks, each a call of its own: the state and the conv ring pass
  // from one segment to the next as between two calls (ring head advanced
  // by the segment's tokens), and the chunks are the ones a single call
  // would form, so the results are the same.
  const long max_rows = ((1L << 31) - 1) / (static_cast<long>(qkv_stride) * 2) / 64 * 64;
  if (T > max_rows) {
    AILA_REQUIRE(max_rows >= 64, "deltanet_layer_prefill: qkv_stride=%d leaves no 64-row chunk in 2 GiB",
                 qkv_stride);
    for (int bb = 0; bb < B; ++bb) {
      for (long t0 = 0; t0 < T; t0 += max_rows) {
        const int ts = static_cast<int>(std::min<long>(max_rows, T - t0));
        const size_t row = static_cast<size_t>(bb) * T + t0;
        const int rc = aila_hip_deltanet_layer_prefill(
            static_cast<const bf16*>(qkv) + row * qkv_stride, qkv_stride, static_cast<const bf16*>(z) + row * z_stride,
            z_stride, static_cast<const bf16*>(a) + row * ab_stride, static_cast<const bf16*>(b) + row * ab_stride,
            ab_stride, conv_w, conv_state + static_cast<size_t>(bb) * kRows * ch,
            static_cast<int>((conv_head + t0) % kRows), dt_bias, A_log, norm_w,
            state + static_cast<size_t>(bb) * Hv * kD * kD, static_cast<bf16*>(out) + row * Hv * kD, workspace,
            workspace_bytes, 1, ts, Hk, Hv, dk, dv, conv_kernel, eps, scale, stream);
        if (rc != AILA_HIP_OK) return rc;
      }
    }
    return AILA_HIP_OK;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int head = ((conv_head % kRows) + kRows) % kRows;
  const ConvIn cv{static_cast<const bf16*>(qkv), qkv_stride, static_cast<const bf16*>(conv_w), conv_state, head, ch};
  launch_deltanet_chunked(nullptr, nullptr, nullptr, &cv, static_cast<const bf16*>(a), static_cast<const bf16*>(b),
                          ab_stride, static_cast<const bf16*>(dt_bias), A_log, state, static_cast<bf16*>(out),
                          static_cast<unsigned char*>(workspace), B, T, Hk, Hv, eps, scale, st);
  const long rows = static_cast<long>(B) * T * Hv;
  const int gate_blocks = static_cast<int>((rows + kGateRows - 1) / kGateRows);
  const int ring_blocks = static_cast<int>((static_cast<long>(B) * kRows * ch + 255) / 256);
  hipLaunchKernelGGL(deltanet_gate_kernel, dim3(static_cast<unsigned>(gate_blocks + ring_blocks)), dim3(256), 0, st,
                     static_cast<bf16*>(out), static_cast<const bf16*>(z), z_stride, norm_w, rows, Hv, eps,
                     gate_blocks, static_cast<const bf16*>(qkv), qkv_stride, conv_state, head, T, ch, B);
  return check_launch("deltanet_layer_prefill");
}

extern "C" int aila_hip_deltanet_layer_decode(const void* qkv, int qkv_stride, const void* z, int z_stride,
                                              const void* a, const void* b, int ab_stride, const void* conv_w,
                                              float* conv_state, int conv_head, const int* conv_heads,
                                              const void* dt_bias, const float* A_log, const float* norm_w,
                                              float* state, void* out, int B, int Hk, int Hv, int dk, int dv,
                                              int conv_kernel, float eps, float scale, unsigned int* arrivals,
                                              void* stream) {
  using namespace aila;
  AILA_REQUIRE(qkv && z && a && b && conv_w && conv_state && norm_w && state && out,
               "deltanet_layer_decode: null pointer");
  AILA_REQUIRE(B > 0 && B <= 65535 && Hk > 0 && Hv > 0 && dk > 0 && dv > 0 && conv_kernel >= 1,
               "deltanet_layer_decode: bad shape (B=%d Hk=%d Hv=%d dk=%d dv=%d K=%d)", B, Hk, Hv, dk, dv,
               conv_kernel);
  const int ch = 2 * Hk * dk + Hv * dv;
  AILA_REQUIRE(qkv_stride >= ch && z_stride >= Hv * dv && ab_stride >= Hv,
               "deltanet_layer_decode: row strides too small (qkv %d < %d, z %d, ab %d)", qkv_stride, ch,
               z_stride, ab_stride);
  if (!(dk == kD && dv == kD && conv_kernel == kConvK && Hv % Hk == 0 &&
        (Hv / Hk == 1 || Hv / Hk == 2 || Hv / Hk == 4))) {
    // general shapes: one token of the sequential layer kernel, then the
    // ring rewrite
    GenericDeltaNet g{};
    g.layer = 1;
    g.qkv = static_cast<const bf16*>(qkv);
    g.qkv_stride = qkv_stride;
    g.z = static_cast<const bf16*>(z);
    g.z_stride = z_stride;
    g.conv_w = static_cast<const bf16*>(conv_w);
    g.conv_state = conv_state;
    g.conv_head = conv_head;
    g.conv_heads = conv_heads;
    g.K = conv_kernel;
    g.norm_w = norm_w;
    g.a = static_cast<const bf16*>(a);
    g.b = static_cast<const bf16*>(b);
    g.ab_stride = ab_stride;
    g.dt_bias = static_cast<const bf16*>(dt_bias);
    g.A_log = A_log;
    g.state = state;
    g.out = static_cast<bf16*>(out);
    g.B = B, g.T = 1, g.Hk = Hk, g.Hv = Hv, g.dk = dk, g.dv = dv;
    g.eps = eps, g.scale = scale;
    return deltanet_generic_launch(g, static_cast<hipStream_t>(stream), "deltanet_layer_decode");
  }
  AILA_REQUIRE(aligned(conv_w, 8) && aligned(z, 8) && z_stride % 4 == 0 && aligned(norm_w, 16) &&
                   aligned(state, 16) && aligned(out, 8) && aligned(arrivals, 4),
               "deltanet_layer_decode: misaligned conv_w/z/norm_w/state/out/arrivals");
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
#define AILA_LAYER_DECODE_VH(GG)                                                                           \
  hipLaunchKernelGGL((deltanet_layer_decode_vh_kernel<GG, 256>), dim3(Hv, B), dim3(256), 0, st, qp, qkv_stride, zp, \
                     z_stride, ap, bp, ab_stride, wp, conv_state, conv_head, conv_heads, dtp, A_log, norm_w,  \
                     state, op, Hk, eps, scale, arrivals)
  // With an arrivals array and G > 1, one workgroup per value head (more
  // workgroups in flight); otherwise one per key head.
  if (arrivals != nullptr && G > 1) {
    switch (G) {
      case 2: AILA_LAYER_DECODE_VH(2); break;
      case 4: AILA_LAYER_DECODE_VH(4); break;
      default:
        return set_error(AILA_HIP_EUNSUPPORTED, "deltanet_layer_decode: Hv/Hk = %d not in {1,2,4}", G);
    }
  } else {
    switch (G) {
      case 1: AILA_LAYER_DECODE(1); break;
      case 2: AILA_LAYER_DECODE(2); break;
      case 4: AILA_LAYER_DECODE(4); break;
      default:
        return set_error(AILA_HIP_EUNSUPPORTED, "deltanet_layer_decode: Hv/Hk = %d not in {1,2,4}", G);
    }
  }
#undef AILA_LAYER_DECODE
#undef AILA_LAYER_DECODE_VH
  return check_launch("deltanet_layer_decode");
}

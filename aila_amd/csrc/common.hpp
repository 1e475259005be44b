// Shared device helpers for the gfx950 kernels: bf16 storage type and
// conversions, MFMA operand vector types, DPP row reductions and the
// C-ABI error plumbing used by every entry point.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <stdint.h>
#include <math.h>

#include "aila_hip.h"

namespace aila {

// bf16 is carried as its 16-bit pattern; arithmetic is always fp32.
typedef uint16_t bf16;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float bf2f(bf16 h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (quiet NaN preserved), identical to
// the host oracle's orc_f32_to_bf16.
__device__ __forceinline__ bf16 f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu))
    return static_cast<bf16>((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<bf16>(u >> 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16x2 (low half = a), round-to-nearest-even in one
// v_cvt_pk_bf16_f32 (same results as f2bf for every non-NaN input).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const f32x2 f = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

// Unpack 8 bf16 held in a 16-byte vector into fp32.
__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(v[i] << 16);
    f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const u32x4& v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// D = A * B + C with A 16x32, B 32x16 (bf16), C/D 16x16 fp32.
// Lane l supplies A[l%16][8*(l/16) .. +8] and B[8*(l/16) .. +8][l%16];
// it receives D[4*(l/16) + j][l%16] in element j.
__device__ __forceinline__ f32x4 mfma16x16x32(const bf16x8_t& a,
                                              const bf16x8_t& b,
                                              const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---- DPP reductions inside a row of 16 lanes ---------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(
      0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

// After these four steps every lane of a 16-lane row holds the row's
// max / sum (each step pairs every lane with a lane of the other half of
// the group being merged).
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp_f<kDppQuadXor1>(x));
  x = fmaxf(x, dpp_f<kDppQuadXor2>(x));
  x = fmaxf(x, dpp_f<kDppRowHalfMirror>(x));
  x = fmaxf(x, dpp_f<kDppRowMirror>(x));
  return x;
}
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f<kDppQuadXor1>(x);
  x += dpp_f<kDppQuadXor2>(x);
  x += dpp_f<kDppRowHalfMirror>(x);
  x += dpp_f<kDppRowMirror>(x);
  return x;
}

// Full 64-lane sum (DPP inside rows, then cross-row swizzles).
__device__ __forceinline__ float wave_sum(float x) {
  x = row16_sum(x);
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// Max over the four lanes {l % 16 + 16 g : g = 0..3} (the same position in
// each 16-lane row), left in every lane: v_permlane32_swap pairs lane l with
// l ^ 32, then v_permlane16_swap pairs rows 0/1 and 2/3. No LDS traffic.
__device__ __forceinline__ float xrow4_max(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xrow4_sum(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// softplus with the reference's +-20 cut-offs (Qwen35HybridTextBackend.cpp:128-132).
__device__ __forceinline__ float softplus_f(float x) {
  if (x > 20.0f) return x;
  if (x < -20.0f) return expf(x);
  return log1pf(expf(x));
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float readlane_f(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}


// ---- LDS DMA and scheduling helpers ---------------------------------------
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16_t;

// Buffer resource word 3 for raw (untyped, unswizzled) gfx9 buffer loads.
constexpr int kBufferRsrcWord3 = 0x00020000;

// Workgroup barrier that orders LDS accesses only (no wait for outstanding
// global loads or LDS DMAs).
__device__ __forceinline__ void phase_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Raw buffer resource (gfx9 layout): 48-bit base, stride 0, num_records in
// bytes, word 3 = untyped raw access. Loads past num_records return zeros.
__device__ __forceinline__ u32x4 buffer_rsrc(const void* base, int num_bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return u32x4{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xFFFFu,
               static_cast<uint32_t>(num_bytes), static_cast<uint32_t>(kBufferRsrcWord3)};
}

// One wave-wide 16-byte-per-lane buffer load written straight to LDS: lane l
// lands at lds + 16*l (the wave's KiB is contiguous). Issued as inline asm so
// the compiler does not treat the LDS tiles as pending DMA targets (it would
// wait for every DMA in flight before any LDS read); kernels order these
// writes themselves with counted vmcnt waits and barriers. M0 is a reserved
// register: it is saved and restored around the load.
__device__ __forceinline__ void dma16_to_lds_at(const u32x4& rsrc, int voffset, uint32_t m0) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
               "buffer_load_dwordx4 %1, %2, 0 offen lds\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(voffset), "s"(rsrc), "s"(m0)
               : "memory");
}
__device__ __forceinline__ void dma16_to_lds(const u32x4& rsrc, int voffset, void* lds) {
  dma16_to_lds_at(rsrc, voffset, static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
}

// s_waitcnt immediate (gfx9 encoding) that waits until at most N vector
// memory operations of this wave are outstanding; expcnt and lgkmcnt are
// left at their maxima (not waited on).
template <int N>
constexpr int vmcnt_imm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  return (N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8);
}

// Transposing LDS read: within each 16-lane group, lane i addresses 4 bf16
// (8 bytes) of row (base + i/4) at column (c0 + 4*(i%4)); lane j receives
// element j of those four rows, i.e. M[base + r][c0 + j] for r = 0..3.
__device__ __forceinline__ u32x2 ds_read_tr4(const void* lds_addr) {
  const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)lds_addr);
  return __builtin_bit_cast(u32x2, v);
}

// Layer prefill input of the DeltaNet chunk prep: the chunk's q, k, v are
// the causal conv1d (4 taps) + SiLU of fused [q | k | v | ...] token rows,
// formed by the prep itself.
struct ConvIn {
  const bf16* qkv;     // [B, T, stride] bf16
  int stride;          // elements per token row
  const bf16* w;       // [ch, 4] taps
  const float* ring;   // [B, 3, ch] fp32 raw rows before token 0
  int head;            // ring row holding token -3 (mod 3)
  int ch;              // channels of a row's [q | k | v] part
};

// ---- rotary positions (text shift and interleaved mRoPE) -----------------
// The device copy of aila_hip_rope_pos, passed by value as a kernel argument
// (a zero struct = rotate at the cache row). Reference:
// ops::apply_rope_partial and the decode_prepare_*_partial rotary_position
// lambda, src/ops/ElementwiseOps.cpp:33-103, 555-863.
typedef aila_hip_rope_pos RopePos;

// Positions of the token in cache row `row` of sequence b: the scalar
// position (row, shifted by the text delta past the prompt) and the three
// mRoPE stream values (all equal to the scalar unless the row lies inside a
// prompt that carries position streams).
struct RowPos {
  int t, h, w;
  int sec_h, sec_w;
};

__device__ __forceinline__ RowPos rope_row_pos(const RopePos& rp, int b, int row) {
  const int plen = rp.prompt_pos_lens ? rp.prompt_pos_lens[b] : rp.prompt_pos_len;
  const int delta = rp.text_pos_deltas ? rp.text_pos_deltas[b] : rp.text_pos_delta;
  const int scalar = row >= plen ? row + delta : row;
  RowPos p{scalar, scalar, scalar, 0, 0};
  if (rp.interleaved && rp.pos_t && rp.pos_h && rp.pos_w) {
    p.sec_h = rp.mrope_section_h;
    p.sec_w = rp.mrope_section_w;
    if (row < plen) {
      const size_t i = static_cast<size_t>(b) * rp.pos_stride + row;
      p.t = rp.pos_t[i];
      p.h = rp.pos_h[i];
      p.w = rp.pos_w[i];
    }
  }
  return p;
}

// Inverse rotary frequencies 1 / theta^(2j/rot), j < rot/2, formed on the
// host with the power correctly rounded to float (double pow, rounded once)
// and passed by value in the kernel arguments. The device powf is not
// correctly rounded: a frequency one ulp off turns pair j's angle at
// position p by p times that ulp (relative output error ~3e-2 at p = 1M),
// where the reference's formula 1 / pow(theta, 2j/rot) with a correctly
// rounded pow (ElementwiseOps.cpp:80) gives the float the host computes.
constexpr int kMaxRopePairs = 128;   // rot <= D <= 256
struct RopeFreq {
  float f[kMaxRopePairs];
};

inline RopeFreq rope_freq_table(float theta, int rot) {
  thread_local float last_theta = 0.f;
  thread_local int last_rot = 0;
  thread_local RopeFreq last{};
  if (theta != last_theta || rot != last_rot) {
    for (int j = 0; j < rot / 2 && j < kMaxRopePairs; ++j) {
      const float x = (2.0f * static_cast<float>(j)) / static_cast<float>(rot);
      const float p = static_cast<float>(std::pow(static_cast<double>(theta), static_cast<double>(x)));
      last.f[j] = 1.0f / p;
    }
    last_theta = theta;
    last_rot = rot;
  }
  return last;
}

// Inverse frequency of rotary pair j: the caller's table, or the host's.
__device__ __forceinline__ float rope_inv_freq(const RopePos& rp, const RopeFreq& rf, int j) {
  return rp.inv_freq ? rp.inv_freq[j] : rf.f[j];
}

// Position rotating frequency index j (0 <= j < rot/2). Selects on values
// (a branch that returns different members would make the compiler address
// the struct through memory, and it then lives in LDS).
__device__ __forceinline__ float rope_freq_pos(RowPos p, int j) {
  const int m = j % 3, q = j / 3;
  int v = p.t;
  v = (m == 1 && q < p.sec_h) ? p.h : v;
  v = (m == 2 && q < p.sec_w) ? p.w : v;
  return static_cast<float>(v);
}

}  // namespace aila

// ---- host-side error plumbing (defined in capi.hip) ---------------------
namespace aila {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// Copies *rp (NULL: zero struct) after checking its fields; returns 0 or an
// AILA_HIP_EINVAL set_error code.
int load_rope_pos(const aila_hip_rope_pos* rp, RopePos* out, const char* what);
}  // namespace aila

#define AILA_REQUIRE(cond, ...)                                  \
  do {                                                           \
    if (!(cond)) return ::aila::set_error(AILA_HIP_EINVAL, __VA_ARGS__); \
  } while (0)

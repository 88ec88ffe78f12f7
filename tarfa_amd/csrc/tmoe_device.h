// Device-side helpers shared by the tmoe kernels (gfx950, wave64).
//
// bf16 values travel as raw 16-bit patterns; conversions are explicit bit
// operations so the rounding is round-to-nearest-even exactly as torch's
// .to(torch.bfloat16) rounds.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tmoe.h"

namespace tmoe {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN.  Written as a
// select, not a branch: it runs per lane inside hot loops.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rounded = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  const uint32_t quiet = (u >> 16) | 0x40u;
  return (uint16_t)((u & 0x7FFFFFFFu) > 0x7F800000u ? quiet : rounded);
}
// Round an fp32 value to the nearest bf16 value, kept in fp32.
__device__ __forceinline__ float rbf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// 16-byte global loads.  Weight streams are read exactly once per call, so they
// carry the non-temporal hint; small shared vectors (x, activations) do not.
// Pointers read from expert tables are generic; the casts keep these global_load
// (not flat_load) instructions.
typedef __attribute__((address_space(1))) const u32x4 g_u32x4;
__device__ __forceinline__ u32x4 ld_stream(const void* p) {
  return __builtin_nontemporal_load((g_u32x4*)p);
}
__device__ __forceinline__ u32x4 ld16(const void* p) { return *(g_u32x4*)p; }
__device__ __forceinline__ uint32_t ld_stream4(const void* p) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) uint32_t*)p);
}

// Dot of 8 bf16 weights (packed in 4 dwords) with 8 fp32 activations.
__device__ __forceinline__ float dot8(const u32x4 w, const float* x, float acc) {
  acc = fmaf(bf16_lo(w.x), x[0], acc);
  acc = fmaf(bf16_hi(w.x), x[1], acc);
  acc = fmaf(bf16_lo(w.y), x[2], acc);
  acc = fmaf(bf16_hi(w.y), x[3], acc);
  acc = fmaf(bf16_lo(w.z), x[4], acc);
  acc = fmaf(bf16_hi(w.z), x[5], acc);
  acc = fmaf(bf16_lo(w.w), x[6], acc);
  acc = fmaf(bf16_hi(w.w), x[7], acc);
  return acc;
}
// Same with both operands packed bf16.
__device__ __forceinline__ float dot8bb(const u32x4 w, const u32x4 a, float acc) {
  acc = fmaf(bf16_lo(w.x), bf16_lo(a.x), acc);
  acc = fmaf(bf16_hi(w.x), bf16_hi(a.x), acc);
  acc = fmaf(bf16_lo(w.y), bf16_lo(a.y), acc);
  acc = fmaf(bf16_hi(w.y), bf16_hi(a.y), acc);
  acc = fmaf(bf16_lo(w.z), bf16_lo(a.z), acc);
  acc = fmaf(bf16_hi(w.z), bf16_hi(a.z), acc);
  acc = fmaf(bf16_lo(w.w), bf16_lo(a.w), acc);
  acc = fmaf(bf16_hi(w.w), bf16_hi(a.w), acc);
  return acc;
}

// Dot of 8 bf16 weights with 8 bf16 activations, both packed in 4 dwords:
// v_dot2c_f32_bf16 (exact bf16 products, fp32 accumulation), pairs in column order.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2bf(uint32_t w, uint32_t a, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, a), acc, false);
}
__device__ __forceinline__ float dot8p(const u32x4 w, const u32x4 a, float acc) {
  acc = dot2bf(w.x, a.x, acc);
  acc = dot2bf(w.y, a.y, acc);
  acc = dot2bf(w.z, a.z, acc);
  acc = dot2bf(w.w, a.w, acc);
  return acc;
}

// DPP lane moves (gfx9 encodings): quad_perm xor1 / xor2, row_half_mirror, row_mirror.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

// Sum over the 64 lanes of a wave in a fixed order; every lane gets the result.
// Lanes are first summed within each row of 16 (quad xor 1, xor 2, half-row
// mirror, row mirror), then the four row sums are added in row order.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (a + b) + (c + d);
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

__device__ __forceinline__ int wave_min_int(int v) {
  v = min(v, __builtin_amdgcn_mov_dpp(v, kDppXor1, 0xF, 0xF, true) );
  v = min(v, __builtin_amdgcn_mov_dpp(v, kDppXor2, 0xF, 0xF, true));
  v = min(v, __builtin_amdgcn_mov_dpp(v, kDppHalfMirror, 0xF, 0xF, true));
  v = min(v, __builtin_amdgcn_mov_dpp(v, kDppMirror, 0xF, 0xF, true));
  int a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  int c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return min(min(a, b), min(c, d));
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppXor1, 0xF, 0xF, true);
  v += (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppXor2, 0xF, 0xF, true);
  v += (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppHalfMirror, 0xF, 0xF, true);
  v += (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppMirror, 0xF, 0xF, true);
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 0) + (uint32_t)__builtin_amdgcn_readlane((int)v, 16) +
         (uint32_t)__builtin_amdgcn_readlane((int)v, 32) + (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
}

// Lane L of v takes the wave-uniform value s (v_writelane_b32).
template <int L>
__device__ __forceinline__ int set_lane(int v, int s) {
  const int su = __builtin_amdgcn_readfirstlane(s);   // the value is wave-uniform; make it scalar
  asm volatile("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(su), "n"(L));
  return v;
}
// Lanes 0..7 take vals[0..7] (wave-uniform values).
__device__ __forceinline__ int spread8(const int (&vals)[8]) {
  int v = 0;
  v = set_lane<0>(v, vals[0]);
  v = set_lane<1>(v, vals[1]);
  v = set_lane<2>(v, vals[2]);
  v = set_lane<3>(v, vals[3]);
  v = set_lane<4>(v, vals[4]);
  v = set_lane<5>(v, vals[5]);
  v = set_lane<6>(v, vals[6]);
  v = set_lane<7>(v, vals[7]);
  return v;
}
// Lanes 0..N-1 take vals[0..N-1] (wave-uniform values).
template <int N, int L = 0>
__device__ __forceinline__ int spread_from(int v, const int (&vals)[N]) {
  if constexpr (L == N) {
    return v;
  } else {
    return spread_from<N, L + 1>(set_lane<L>(v, vals[L]), vals);
  }
}
template <int N>
__device__ __forceinline__ int spread(const int (&vals)[N]) {
  return spread_from<N, 0>(0, vals);
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }
__device__ __forceinline__ float sigmoid_f32(float z) { return 1.0f / (1.0f + expf(-z)); }

// SwiGLU activation at the reference's bf16 rounding points:
// bf16(bf16(silu(g)) * u) with g, u already bf16 values.
__device__ __forceinline__ float swiglu_bf16(float g, float u) { return rbf16(rbf16(silu_f32(g)) * u); }
// The same rounding points from two fp32 accumulators, as bf16 bits: the conversions are
// the hardware's (v_cvt_pk_bf16_f32, round to nearest even like f32_to_bf16 for every value
// but NaN payloads) and silu is g * rcp(1 + e^-g) (the hardware reciprocal, within ~1 ulp of
// fp32 g / (1 + e^-g)).  The prefill GEMM epilogue's form, where an IEEE division and
// software rounding would hold up the weight stream.
typedef __bf16 bf16x2_hw __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t swiglu_bits_hw(float gacc, float uacc) {
  const uint32_t gu = __builtin_bit_cast(uint32_t, bf16x2_hw{(__bf16)gacc, (__bf16)uacc});
  const float g = __uint_as_float(gu << 16), u = __uint_as_float(gu & 0xFFFF0000u);
  const float s = (float)(__bf16)(g * __builtin_amdgcn_rcpf(1.0f + expf(-g)));
  return __builtin_bit_cast(uint16_t, (__bf16)(s * u));
}
// Two fp32 values to bf16 bits in one hardware conversion (v_cvt_pk_bf16_f32: round to nearest
// even, as f32_to_bf16, for every value but NaN payloads; low half: a).
__device__ __forceinline__ uint32_t bf16x2_bits_hw(float a, float b) {
  return __builtin_bit_cast(uint32_t, bf16x2_hw{(__bf16)a, (__bf16)b});
}
// Round a and b to the nearest bf16 values, in place (rbf16 of each, one conversion).
__device__ __forceinline__ void rbf16x2_hw(float& a, float& b) {
  const uint32_t w = bf16x2_bits_hw(a, b);
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xFFFF0000u);
}

}  // namespace tmoe

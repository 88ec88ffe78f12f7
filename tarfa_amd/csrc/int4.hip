// Int4 fast-mode weight format: quantise and dequantise (debug materialisation), and the
// reference's own fp16 dequantisation of its per-row-scale files.
//
// Format (a group-scaled form of the reference's per-row int4 layout,
// tarfa/engine/channel_q4.py:10-14, tarfa/engine/moe_kernel.py:110-114):
//   packed [N, K/2] uint8   low nibble = even k, high nibble = odd k, value = nibble - 8
//   scales [N, K/G] bf16    one scale per (row, group of G consecutive k)
//   dequant  w_hat = bf16((nibble - 8) * s[n, k / G])   (the product is exact in fp32)
// The reference ships no quantiser; this build's is
//   s = bf16(max_{k in group} |w| / 7)       IEEE fp32 division, round to nearest even
//   q = clamp(rint(w / s), -8, 7)            rint rounds half to even; s == 0 gives q = 0
// Every step is one correctly rounded IEEE operation, so the device matches the
// host restatement bit for bit.
#include "tmoe_device.h"

namespace tmoe {

// One wave per (row, group): lanes stride the group's columns.  G is a multiple
// of 2 and at most 2048.
__global__ __launch_bounds__(256) void k_quantize_int4(const uint16_t* __restrict__ w, int N, int K, int G,
                                                       uint8_t* __restrict__ packed, uint16_t* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const long unit = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int groups = K / G;
  if (unit >= (long)N * groups) return;
  const int n = (int)(unit / groups), g = (int)(unit % groups);
  const uint16_t* row = w + (size_t)n * K + (size_t)g * G;
  float amax = 0.f;
  for (int c = lane; c < G; c += 64) amax = fmaxf(amax, fabsf(bf16_to_f32(row[c])));
  // max over the wave (order-free)
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  const float s = rbf16(amax / 7.0f);
  if (lane == 0) scales[(size_t)n * groups + g] = f32_to_bf16(s);
  uint8_t* prow = packed + (size_t)n * (K / 2) + (size_t)g * (G / 2);
  for (int c = 2 * lane; c < G; c += 128) {
    int q[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float r = s == 0.f ? 0.f : rintf(bf16_to_f32(row[c + j]) / s);
      q[j] = (int)fminf(fmaxf(r, -8.f), 7.f);
    }
    prow[c / 2] = (uint8_t)((q[0] + 8) | ((q[1] + 8) << 4));
  }
}

// Eight dequantised values (16 bytes out) per thread per iteration.
__global__ __launch_bounds__(256) void k_dequant_int4(const uint8_t* __restrict__ packed,
                                                      const uint16_t* __restrict__ scales, int N, int K, int G,
                                                      uint16_t* __restrict__ out) {
  const size_t total = (size_t)N * K / 8;
  for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < total; u += (size_t)gridDim.x * blockDim.x) {
    const size_t e0 = u * 8;
    const int n = (int)(e0 / K), k0 = (int)(e0 % K);
    const uint32_t word = *reinterpret_cast<const uint32_t*>(packed + (size_t)n * (K / 2) + k0 / 2);
    uint16_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int q = (int)((word >> (4 * j)) & 0xFu) - 8;
      const float s = bf16_to_f32(scales[(size_t)n * (K / G) + (k0 + j) / G]);
      v[j] = f32_to_bf16((float)q * s);
    }
    u32x4 pk;
    pk.x = v[0] | ((uint32_t)v[1] << 16);
    pk.y = v[2] | ((uint32_t)v[3] << 16);
    pk.z = v[4] | ((uint32_t)v[5] << 16);
    pk.w = v[6] | ((uint32_t)v[7] << 16);
    *reinterpret_cast<u32x4*>(out + e0) = pk;
  }
}

// The reference's own dequantisation (tarfa/engine/channel_q4.py:10-14,
// moe_kernel.py:110-114): fp16 scales, fp16 result, w = fp16((nibble - 8) * s[n, k / G]).
// The product of a 4-bit integer and an 11-bit fp16 significand is exact in fp32, so one
// round-to-nearest-even conversion to fp16 (subnormals kept) gives torch's fp16 multiply.
// With G = K the scale is per row, the reference's layout.
__global__ __launch_bounds__(256) void k_dequant_int4_f16(const uint8_t* __restrict__ packed,
                                                          const uint16_t* __restrict__ scales, int N, int K, int G,
                                                          uint16_t* __restrict__ out) {
  const size_t total = (size_t)N * K / 8;
  for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < total; u += (size_t)gridDim.x * blockDim.x) {
    const size_t e0 = u * 8;
    const int n = (int)(e0 / K), k0 = (int)(e0 % K);
    const uint32_t word = *reinterpret_cast<const uint32_t*>(packed + (size_t)n * (K / 2) + k0 / 2);
    uint16_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int q = (int)((word >> (4 * j)) & 0xFu) - 8;
      const float s = (float)__builtin_bit_cast(_Float16, scales[(size_t)n * (K / G) + (k0 + j) / G]);
      v[j] = __builtin_bit_cast(uint16_t, (_Float16)((float)q * s));
    }
    u32x4 pk;
    pk.x = v[0] | ((uint32_t)v[1] << 16);
    pk.y = v[2] | ((uint32_t)v[3] << 16);
    pk.z = v[4] | ((uint32_t)v[5] << 16);
    pk.w = v[6] | ((uint32_t)v[7] << 16);
    *reinterpret_cast<u32x4*>(out + e0) = pk;
  }
}

}  // namespace tmoe

using namespace tmoe;

static int check_q4(const void* a, const void* b, int N, int K, int G) {
  if (!a || !b) return TMOE_ERR_NULL;
  if (N < 1 || K < 8 || K % 8 || G < 2 || G > 2048 || G % 2 || K % G) return TMOE_ERR_SHAPE;
  return TMOE_OK;
}

extern "C" int tmoe_quantize_int4(const void* w, int N, int K, int G, void* packed, void* scales, void* stream) {
  if (int st = check_q4(w, packed, N, K, G)) return st;
  if (!scales) return TMOE_ERR_NULL;
  const long units = (long)N * (K / G);
  const int blocks = (int)((units + 3) / 4);
  hipLaunchKernelGGL(k_quantize_int4, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint16_t*)w, N, K, G,
                     (uint8_t*)packed, (uint16_t*)scales);
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

extern "C" int tmoe_dequant_int4_bf16(const void* packed, const void* scales, int N, int K, int G, void* out,
                                      void* stream) {
  if (int st = check_q4(packed, out, N, K, G)) return st;
  if (!scales) return TMOE_ERR_NULL;
  if (((uintptr_t)packed & 3u) || ((uintptr_t)out & 15u)) return TMOE_ERR_ALIGN;
  const size_t units = (size_t)N * K / 8;
  const int blocks = (int)((units + 255) / 256 < 4096 ? (units + 255) / 256 : 4096);
  hipLaunchKernelGGL(k_dequant_int4, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)packed,
                     (const uint16_t*)scales, N, K, G, (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

extern "C" int tmoe_dequant_int4_f16(const void* packed, const void* scales, int N, int K, int G, void* out,
                                     void* stream) {
  if (!packed || !out || !scales) return TMOE_ERR_NULL;
  if (N < 1 || K < 8 || K % 8 || G < 2 || G % 2 || K % G) return TMOE_ERR_SHAPE;
  if (((uintptr_t)packed & 3u) || ((uintptr_t)out & 15u)) return TMOE_ERR_ALIGN;
  const size_t units = (size_t)N * K / 8;
  const int blocks = (int)((units + 255) / 256 < 4096 ? (units + 255) / 256 : 4096);
  hipLaunchKernelGGL(k_dequant_int4_f16, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)packed,
                     (const uint16_t*)scales, N, K, G, (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

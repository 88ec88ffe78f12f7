// Seeded, counter-based fill of bf16 / fp32 tensors on the device.
//
// Element i of a tensor with key K is a pure function of (K, start + i):
//   h_i = mix(K + (i + 1) * 0x9E3779B97F4A7C15)       splitmix64 output function
//   bf16: c = sum of the twelve 16-bit fields of h_{3i}, h_{3i+1}, h_{3i+2} - 393210 (exact int),
//         value = bf16(fp32(c) * scale)                 one fp32 rounding, then RNE
//   fp32: c = sum of the twelve 32-bit fields of h_{6i} .. h_{6i+5} - 6*(2^32-1) (exact int64),
//         value = fp32(double(c) * scale)               one fp64 rounding, then RNE to fp32
// (Irwin-Hall n = 12: the classical sum-of-twelve-uniforms normal, bounded at +-6 sigma.)
// Integer sums, int->float conversions of exactly representable integers and
// single IEEE multiplies round identically on host and device, so the host can
// regenerate any slab bit-for-bit.  The whole-model weight set (~194 GB at
// H=2560, E=256, I=1024, 48 layers) is written here in HBM, never on the host.
#include "tmoe_device.h"

namespace tmoe {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t hash_at(uint64_t key, uint64_t i) {
  return mix64(key + (i + 1ull) * 0x9E3779B97F4A7C15ull);
}

// Eight bf16 values (16 bytes) per thread per iteration; grid-stride loop.
__global__ __launch_bounds__(256) void k_fill_bf16(uint16_t* __restrict__ dst, uint64_t n, uint64_t key,
                                                   float scale, uint64_t start) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x * 8ull;
  for (uint64_t base = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8ull; base < n; base += stride) {
    uint16_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint64_t i3 = 3ull * (start + base + j);
      int32_t c = -393210;
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const uint64_t h = hash_at(key, i3 + q);
        c += (int32_t)((h & 0xFFFF) + ((h >> 16) & 0xFFFF) + ((h >> 32) & 0xFFFF) + (h >> 48));
      }
      v[j] = f32_to_bf16((float)c * scale);
    }
    if (base + 8 <= n && (((uintptr_t)(dst + base)) & 15) == 0) {
      u32x4 pk;
      pk.x = v[0] | ((uint32_t)v[1] << 16);
      pk.y = v[2] | ((uint32_t)v[3] << 16);
      pk.z = v[4] | ((uint32_t)v[5] << 16);
      pk.w = v[6] | ((uint32_t)v[7] << 16);
      *reinterpret_cast<u32x4*>(dst + base) = pk;
    } else {
      for (int j = 0; j < 8 && base + j < n; ++j) dst[base + j] = v[j];
    }
  }
}

__global__ __launch_bounds__(256) void k_fill_f32(float* __restrict__ dst, uint64_t n, uint64_t key, double scale,
                                                  uint64_t start) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    int64_t c = -6ll * 0xFFFFFFFFll;
#pragma unroll
    for (int q = 0; q < 6; ++q) {
      const uint64_t h = hash_at(key, 6ull * (start + i) + q);
      c += (int64_t)(h & 0xFFFFFFFFull) + (int64_t)(h >> 32);
    }
    dst[i] = (float)((double)c * scale);
  }
}

static unsigned fill_grid(uint64_t items) {
  const uint64_t blocks = (items + 255) / 256;
  return (unsigned)(blocks < 65536 ? (blocks ? blocks : 1) : 65536);
}

}  // namespace tmoe

extern "C" int tmoe_fill_bf16(void* dst, uint64_t n, uint64_t key, float scale, uint64_t start, void* stream) {
  if (n == 0) return TMOE_OK;
  if (!dst) return TMOE_ERR_NULL;
  hipLaunchKernelGGL(tmoe::k_fill_bf16, dim3(tmoe::fill_grid((n + 7) / 8)), dim3(256), 0, (hipStream_t)stream,
                     (uint16_t*)dst, n, key, scale, start);
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

extern "C" int tmoe_fill_f32(float* dst, uint64_t n, uint64_t key, double scale, uint64_t start, void* stream) {
  if (n == 0) return TMOE_OK;
  if (!dst) return TMOE_ERR_NULL;
  hipLaunchKernelGGL(tmoe::k_fill_f32, dim3(tmoe::fill_grid(n)), dim3(256), 0, (hipStream_t)stream, dst, n, key,
                     scale, start);
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

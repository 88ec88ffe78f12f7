// The steps on either side of the MoE block in a Qwen3.5-MoE decoder layer
// (transformers modeling_qwen3_5_moe.py:870-875): the post-attention RMSNorm that
// produces the block's input, and the residual add of its output.
//   x   = bf16(h * (1 / sqrt(mean(h^2) + eps)) * (1 + w))   in fp32 (:806-814)
//   out = bf16(h + y)                                          (:875)
// The fused decode kernel forms x in every task that loads it and adds the residual in
// its combine; the prefill adds it in its combine.  These kernels serve the other paths:
// x for T > 1 (once, read by the router, the shared gate and the GEMMs) and the residual
// add after the unfused decode.
#include <hip/hip_runtime.h>

#include "tmoe.h"
#include "tmoe_gemv.h"

namespace tmoe {

// One wave per row (H <= 4096: MAXC 512-column chunks per lane).
template <int MAXC>
__global__ __launch_bounds__(256) void k_rmsnorm(const uint16_t* __restrict__ h, const uint16_t* __restrict__ w,
                                                 float eps, int T, int H, uint16_t* __restrict__ x) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  XPack<MAXC> f;
  load_xpack_norm<MAXC, false>(f, h + (size_t)t * H, w, eps, H, lane);
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int col = c * 512 + lane * 8;
    if (col < H) *reinterpret_cast<u32x4*>(x + (size_t)t * H + col) = f.v[c];
  }
}

__global__ __launch_bounds__(256) void k_residual_add(const uint16_t* __restrict__ h, uint16_t* __restrict__ y,
                                                      size_t n) {
  const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i >= n) return;
  const u32x4 a = ld16(h + i), b = ld16(y + i);
  const uint32_t ha[4] = {a.x, a.y, a.z, a.w}, yb[4] = {b.x, b.y, b.z, b.w};
  uint32_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    o[q] = (uint32_t)f32_to_bf16(bf16_lo(ha[q]) + bf16_lo(yb[q])) |
           ((uint32_t)f32_to_bf16(bf16_hi(ha[q]) + bf16_hi(yb[q])) << 16);
  *reinterpret_cast<u32x4*>(y + i) = u32x4{o[0], o[1], o[2], o[3]};
}

int rmsnorm_launch(const uint16_t* h, const uint16_t* w, float eps, int T, int H, uint16_t* x, hipStream_t s) {
  const dim3 g((T + 3) / 4), b(256);
  const int nc = (H + 511) / 512;
  switch (nc <= 2 ? 2 : nc <= 4 ? 4 : nc <= 6 ? 6 : 8) {
    case 2: hipLaunchKernelGGL(k_rmsnorm<2>, g, b, 0, s, h, w, eps, T, H, x); break;
    case 4: hipLaunchKernelGGL(k_rmsnorm<4>, g, b, 0, s, h, w, eps, T, H, x); break;
    case 6: hipLaunchKernelGGL(k_rmsnorm<6>, g, b, 0, s, h, w, eps, T, H, x); break;
    default: hipLaunchKernelGGL(k_rmsnorm<8>, g, b, 0, s, h, w, eps, T, H, x); break;
  }
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

// y := bf16(h + y) over n elements (n a multiple of 8, 16-byte aligned buffers).
int residual_add_launch(const uint16_t* h, uint16_t* y, size_t n, hipStream_t s) {
  if (n == 0) return TMOE_OK;
  hipLaunchKernelGGL(k_residual_add, dim3((unsigned)((n / 8 + 255) / 256)), dim3(256), 0, s, h, y, n);
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

}  // namespace tmoe

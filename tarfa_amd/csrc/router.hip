// Router for T tokens: fp32 logits GEMV (when logits are not supplied) and a
// one-wave-per-token softmax / top-k / renormalise.
//   transformers/.../modeling_qwen3_5_moe.py:768-776 (Qwen3_5MoeTopKRouter.forward),
//   with fp32 logits in place of the hidden-dtype F.linear at :770.
#include <stdlib.h>

#include "tmoe_gemv.h"
#include "tmoe_ws.h"

namespace tmoe {

constexpr int kRouterMfmaFrom = 128;   // tokens from which the logits run as an MFMA GEMM (equal at 32..128)

// logits[t, e] = sum_h x[t, h] * wg[e, h] in fp32.  Block (t, y) of a (T, Y) grid: wave w
// handles experts 16 y + 4 w .. + 3, then 16 (y + Y) + 4 w, ... (4 rows in flight per
// wave).  Few tokens take Y = E / 16 (one round trip per wave), many take Y = 1.
template <int MAXC>
__global__ __launch_bounds__(256) void k_router_logits(const uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ wg, int H, int E,
                                                       float* __restrict__ logits) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int t = blockIdx.x;
  XFrag<MAXC> xf;
  load_xfrag<MAXC>(xf, x + (size_t)t * H, H, lane);
  for (int e0 = (int)blockIdx.y * 16 + wid * 4; e0 < E; e0 += 16 * (int)gridDim.y) {
    const uint16_t* rows[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) rows[r] = wg + (size_t)min(e0 + r, E - 1) * H;
    float d[4];
    wave_dots<MAXC, 4>(rows, xf, H, lane, d);
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (e0 + r < E) logits[(size_t)t * E + e0 + r] = d[r];
    }
  }
}

// The same logits for many tokens as a GEMM on the matrix cores: v_mfma_f32_16x16x32_bf16
// (exact bf16 products, fp32 accumulation).  Block (tb, eb) of 4 waves computes tokens
// 32 tb .. + 31 x experts 32 eb .. + 31 (four 16 x 16 blocks); the K steps (32 wide) are
// dealt round-robin to the 4 waves (step s to wave s % 4), and the waves' partial sums are
// added through LDS in wave order, so each logit is one fixed-order fp32 sum.  Operand
// fragments come straight from memory, lane l holding row l % 16 and k = 8 (l / 16) .. + 7
// of a step (16 bytes), for the token rows (A) and the router rows (B); rows past T or E
// repeat the last one and are never stored.  The GEMV form above reads the whole router
// weight once per token (1.3 GB of L2 reads per 1000 tokens at H = 2560, E = 256); this
// reads it once per 32 tokens.  H a multiple of 32.
typedef __bf16 rt_bf16x8 __attribute__((ext_vector_type(8)));
constexpr int kRtUnroll = 8;   // k steps of a wave whose loads are issued together
__global__ __launch_bounds__(256) void k_router_logits_mfma(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ wg, int T, int H, int E,
                                                            float* __restrict__ logits) {
  __shared__ f32x4 red[4][4][64];   // [wave][block (i, j)][lane]
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int t0 = (int)blockIdx.x * 32, e0 = (int)blockIdx.y * 32;
  const int r = lane & 15, kq = (lane >> 4) * 8;
  const uint16_t* pa[2];
  const uint16_t* pb[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    pa[i] = x + (size_t)min(t0 + 16 * i + r, T - 1) * H + kq;
    pb[i] = wg + (size_t)min(e0 + 16 * i + r, E - 1) * H + kq;
  }
  f32x4 c[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) c[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto step = [&](const u32x4 (&a)[2], const u32x4 (&b)[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        c[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(rt_bf16x8, a[i]),
                                                          __builtin_bit_cast(rt_bf16x8, b[j]), c[i][j], 0, 0, 0);
  };
  const int nsteps = H / 32;
  int st = wid;
  for (; st + 4 * (kRtUnroll - 1) < nsteps; st += 4 * kRtUnroll) {
    u32x4 a[kRtUnroll][2], b[kRtUnroll][2];
#pragma unroll
    for (int u = 0; u < kRtUnroll; ++u)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        a[u][i] = ld16(pa[i] + 32 * (st + 4 * u));
        b[u][i] = ld16(pb[i] + 32 * (st + 4 * u));
      }
#pragma unroll
    for (int u = 0; u < kRtUnroll; ++u) step(a[u], b[u]);
  }
  for (; st < nsteps; st += 4) {
    u32x4 a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      a[i] = ld16(pa[i] + 32 * st);
      b[i] = ld16(pb[i] + 32 * st);
    }
    step(a, b);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) red[wid][2 * i + j][lane] = c[i][j];
  __syncthreads();
  // Wave w stores block (i, j) = (w / 2, w % 2): lane l holds tokens 16 i + 4 (l / 16) + q,
  // expert 16 j + l % 16.
  const int i = wid >> 1, j = wid & 1;
  const f32x4 v = ((red[0][wid][lane] + red[1][wid][lane]) + red[2][wid][lane]) + red[3][wid][lane];
  const int e = e0 + 16 * j + r;
  if (e < E) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int t = t0 + 16 * i + 4 * (lane >> 4) + q;
      if (t < T) logits[(size_t)t * E + e] = v[q];
    }
  }
}

// One wave per token.
template <int MAXEPL>
__global__ __launch_bounds__(256) void k_router_topk(const float* __restrict__ logits, int T, int E, int k,
                                                     int64_t* ids64, uint16_t* wb, int32_t* ids32, float* wf,
                                                     uint32_t* heat) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  TopkOut o;
  o.ids32 = ids32 ? ids32 + (size_t)t * k : nullptr;
  o.wf = wf ? wf + (size_t)t * k : nullptr;
  o.ids64 = ids64 ? ids64 + (size_t)t * k : nullptr;
  o.wb = wb ? wb + (size_t)t * k : nullptr;
  o.heat = heat;
  wave_topk<MAXEPL>(logits + (size_t)t * E, false, E, k, lane, o);
}

int launch_router_logits(const uint16_t* x, const uint16_t* wg, int T, int H, int E, float* logits,
                         hipStream_t s) {
  static const int mfma_from = [] {
    const char* e = getenv("TMOE_ROUTER_MFMA_FROM");
    return e ? atoi(e) : kRouterMfmaFrom;
  }();
  if (T >= mfma_from && H % 32 == 0) {
    const dim3 g((T + 31) / 32, (E + 31) / 32);
    hipLaunchKernelGGL(k_router_logits_mfma, g, dim3(256), 0, s, x, wg, T, H, E, logits);
    return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
  }
  const int nc = (H + 511) / 512;
  const dim3 g(T, T < 512 ? (E + 15) / 16 : 1);
  switch (nc <= 2 ? 2 : nc <= 4 ? 4 : nc <= 6 ? 6 : 8) {
    case 2: hipLaunchKernelGGL(k_router_logits<2>, g, dim3(256), 0, s, x, wg, H, E, logits); break;
    case 4: hipLaunchKernelGGL(k_router_logits<4>, g, dim3(256), 0, s, x, wg, H, E, logits); break;
    case 6: hipLaunchKernelGGL(k_router_logits<6>, g, dim3(256), 0, s, x, wg, H, E, logits); break;
    default: hipLaunchKernelGGL(k_router_logits<8>, g, dim3(256), 0, s, x, wg, H, E, logits); break;
  }
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

// The same top-k with the shared expert's gate beside it: wave t also computes
// gs[t] = bf16(sigmoid(bf16(x_t . w_sg))) (fp32 products of the bf16 values, lane l summing
// columns 512 c + 8 l .. + 7 over c in order, then the wave sum), its x row and the gate row
// requested before the logits so both round trips overlap: one launch where a separate
// shared-gate GEMV took a second.
template <int MAXEPL, int MAXC>
__global__ __launch_bounds__(256) void k_router_topk_gate(const float* __restrict__ logits, int T, int E, int k,
                                                          int64_t* ids64, uint16_t* wb, int32_t* ids32, float* wf,
                                                          uint32_t* heat, const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ wsg, int H,
                                                          float* __restrict__ gs) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  u32x4 xr[MAXC], w[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int col = c * 512 + lane * 8;
    xr[c] = col < H ? ld16(x + (size_t)t * H + col) : u32x4{0u, 0u, 0u, 0u};
    w[c] = col < H ? ld_stream(wsg + col) : u32x4{0u, 0u, 0u, 0u};
  }
  TopkOut o;
  o.ids32 = ids32 ? ids32 + (size_t)t * k : nullptr;
  o.wf = wf ? wf + (size_t)t * k : nullptr;
  o.ids64 = ids64 ? ids64 + (size_t)t * k : nullptr;
  o.wb = wb ? wb + (size_t)t * k : nullptr;
  o.heat = heat;
  wave_topk<MAXEPL>(logits + (size_t)t * E, false, E, k, lane, o);
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const float xv[8] = {bf16_lo(xr[c].x), bf16_hi(xr[c].x), bf16_lo(xr[c].y), bf16_hi(xr[c].y),
                         bf16_lo(xr[c].z), bf16_hi(xr[c].z), bf16_lo(xr[c].w), bf16_hi(xr[c].w)};
    acc = dot8(w[c], xv, acc);
  }
  const float d = wave_sum(acc);
  if (lane == 0) gs[t] = rbf16(sigmoid_f32(rbf16(d)));
}

int launch_router_topk_gate(const float* logits, int T, int E, int k, int64_t* ids64, uint16_t* wb, int32_t* ids32,
                            float* wf, uint32_t* heat, const uint16_t* x, const uint16_t* w_sg, int H, float* gs,
                            hipStream_t s) {
  const dim3 grid((T + 3) / 4), block(256);
  const bool small_e = (E + 63) / 64 <= 4;
  const int nc = (H + 511) / 512;
#define TMOE_TOPK_GATE(MAXC)                                                                                      \
  if (small_e)                                                                                                    \
    hipLaunchKernelGGL((k_router_topk_gate<4, MAXC>), grid, block, 0, s, logits, T, E, k, ids64, wb, ids32, wf,    \
                       heat, x, w_sg, H, gs);                                                                     \
  else                                                                                                            \
    hipLaunchKernelGGL((k_router_topk_gate<16, MAXC>), grid, block, 0, s, logits, T, E, k, ids64, wb, ids32, wf,   \
                       heat, x, w_sg, H, gs);
  switch (nc <= 2 ? 2 : nc <= 4 ? 4 : nc <= 6 ? 6 : 8) {
    case 2: TMOE_TOPK_GATE(2) break;
    case 4: TMOE_TOPK_GATE(4) break;
    case 6: TMOE_TOPK_GATE(6) break;
    default: TMOE_TOPK_GATE(8) break;
  }
#undef TMOE_TOPK_GATE
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

int launch_router_topk(const float* logits, int T, int E, int k, int64_t* ids64, uint16_t* wb, int32_t* ids32,
                       float* wf, uint32_t* heat, hipStream_t s) {
  const dim3 grid((T + 3) / 4), block(256);
  const int epl = (E + 63) / 64;
  if (epl <= 4)
    hipLaunchKernelGGL(k_router_topk<4>, grid, block, 0, s, logits, T, E, k, ids64, wb, ids32, wf, heat);
  else
    hipLaunchKernelGGL(k_router_topk<16>, grid, block, 0, s, logits, T, E, k, ids64, wb, ids32, wf, heat);
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

// The reference's re-truncation at its experts boundary (tarfa/engine/fused_int4.py:157-160):
// when a token carries more than j routed experts, keep the j largest bf16 weights (equal
// weights keep the lower slot first), gather their ids and renormalise in bf16:
// w'_r = bf16(w_r / bf16(sum of the kept weights)), the sum in fp32 in the kept (descending)
// order.  One thread per token; k <= 16.
__global__ __launch_bounds__(256) void k_topk_renorm(const int64_t* __restrict__ ids,
                                                     const uint16_t* __restrict__ w, int T, int k, int j,
                                                     int64_t* __restrict__ ids_out, uint16_t* __restrict__ w_out) {
  const int t = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (t >= T) return;
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = i < k ? bf16_to_f32(w[(size_t)t * k + i]) : -INFINITY;
  uint32_t used = 0;
  int sel[16];
  float sum = 0.f;
  for (int r = 0; r < j; ++r) {
    int best = -1;
    float bv = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const bool cand = i < k && !((used >> i) & 1u) && (best < 0 || v[i] > bv);
      best = cand ? i : best;
      bv = cand ? v[i] : bv;
    }
    used |= 1u << best;
    sel[r] = best;
    sum += bv;
  }
  const float sb = rbf16(sum);
  for (int r = 0; r < j; ++r) {
    const int i = sel[r];
    ids_out[(size_t)t * j + r] = ids[(size_t)t * k + i];
    w_out[(size_t)t * j + r] = f32_to_bf16(bf16_to_f32(w[(size_t)t * k + i]) / sb);
  }
}

int check_router_shape(int T, int H, int E, int k) {
  if (T < 1 || E < 1 || E > 1024 || k < 1 || k > 16 || k > E) return TMOE_ERR_SHAPE;
  if (H < 8 || H > 4096 || H % 8) return TMOE_ERR_SHAPE;
  return TMOE_OK;
}

}  // namespace tmoe

extern "C" int tmoe_router_topk(const void* x, const void* router_w, const float* logits_in, int T, int H, int E,
                                int k, int64_t* ids_out, void* weights_out, float* logits_out, uint32_t* heat,
                                void* stream) {
  using namespace tmoe;
  if (int st = check_router_shape(T, H, E, k)) return st;
  if (!ids_out || !weights_out) return TMOE_ERR_NULL;
  hipStream_t s = (hipStream_t)stream;
  const float* lg = logits_in;
  if (!lg) {
    if (!x || !router_w || !logits_out) return TMOE_ERR_NULL;   // logits need a home when computed
    if (((uintptr_t)x | (uintptr_t)router_w) & 15) return TMOE_ERR_ALIGN;
    if (int st = launch_router_logits((const uint16_t*)x, (const uint16_t*)router_w, T, H, E, logits_out, s))
      return st;
    lg = logits_out;
  } else if (logits_out && logits_out != logits_in) {
    if (hipMemcpyAsync(logits_out, logits_in, sizeof(float) * (size_t)T * E, hipMemcpyDeviceToDevice, s) !=
        hipSuccess)
      return TMOE_ERR_HIP;
  }
  return launch_router_topk(lg, T, E, k, ids_out, (uint16_t*)weights_out, nullptr, nullptr, heat, s);
}

extern "C" int tmoe_topk_renorm_bf16(const int64_t* ids, const void* weights, int T, int k, int j, int64_t* ids_out,
                                     void* weights_out, void* stream) {
  using namespace tmoe;
  if (T < 1 || k < 1 || k > 16 || j < 1 || j > k) return TMOE_ERR_SHAPE;
  if (!ids || !weights || !ids_out || !weights_out) return TMOE_ERR_NULL;
  hipLaunchKernelGGL(k_topk_renorm, dim3((T + 255) / 256), dim3(256), 0, (hipStream_t)stream, ids,
                     (const uint16_t*)weights, T, k, j, ids_out, (uint16_t*)weights_out);
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

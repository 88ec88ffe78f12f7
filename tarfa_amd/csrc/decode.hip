// Batch-1 (decode) MoE layer: bandwidth-bound bf16 GEMVs streamed as 16-byte
// loads, fp32 accumulation, bf16 rounding at the reference's points.
//
// Three launches, ordered on one stream:
//   A  router logits (fp32) + top-k in the last-arriving block, shared-gate logit,
//      shared expert gate/up + SwiGLU                       [router ~1.3 MB, shared up ~10.5 MB]
//   B  routed gate/up + SwiGLU for the k selected experts (ids read on device),
//      shared expert down + sigmoid-gate scale               [~84 MB + ~5.2 MB]
//   C  routed down for all k experts of each output row, then the router-order
//      bf16 chain and the shared add                          [~42 MB]
// Reference: tarfa/engine/fused_int4.py:163-205 (decode loop :192-194, combine
// :180/:194/:202); transformers/.../modeling_qwen3_5_moe.py:715-717, 787-798.
#include "tmoe_gemv.h"
#include "tmoe_ws.h"
#include "tmoe_decode.h"

namespace tmoe {



constexpr int kPairsPerWave = 2;                  // gate/up row pairs per wave in the up projections
constexpr int kPairsPerBlock = 4 * kPairsPerWave;
constexpr int kDownRowsPerWave = 4;               // shared-down rows per wave
constexpr int kDownRowsPerBlock = 4 * kDownRowsPerWave;

// Expert id of slot j and whether it is computed; flags ids outside [0, E].
__device__ __forceinline__ bool slot_expert(const DecodeParams& p, int j, int& e) {
  e = p.ids_in ? (int)p.ids_in[j] : p.ids_ws[j];
  if (e >= 0 && e < p.E) return true;
  if (e != p.E && p.err) atomicOr(p.err, 1u);   // sentinel E is a silent skip
  return false;
}
__device__ __forceinline__ float slot_weight(const DecodeParams& p, int j) {
  return p.w_in ? bf16_to_f32(p.w_in[j]) : p.w_ws[j];
}

// Gate/up pairs [i0, i0 + kPairsPerWave) of one expert; writes bf16 SwiGLU activations.
template <int MAXC>
__device__ __forceinline__ void up_pairs(const uint16_t* gate, const uint16_t* up, int i0, int n_rows, int K,
                                         const XFrag<MAXC>& xf, int lane, uint16_t* act) {
  const uint16_t* rows[2 * kPairsPerWave];
#pragma unroll
  for (int q = 0; q < kPairsPerWave; ++q) {
    const int i = min(i0 + q, n_rows - 1);
    rows[q] = gate + (size_t)i * K;
    rows[kPairsPerWave + q] = up + (size_t)i * K;
  }
  float d[2 * kPairsPerWave];
  wave_dots<MAXC, 2 * kPairsPerWave>(rows, xf, K, lane, d);
  if (lane == 0) {
#pragma unroll
    for (int q = 0; q < kPairsPerWave; ++q)
      if (i0 + q < n_rows) act[i0 + q] = f32_to_bf16(swiglu_bf16(rbf16(d[q]), rbf16(d[kPairsPerWave + q])));
  }
}

// ---------------------------------------------------------------- A
template <int MAXC>
__global__ __launch_bounds__(256) void k_decode_a(DecodeParams p) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  XFrag<MAXC> xf;
  load_xfrag<MAXC>(xf, p.x, p.H, lane);
  const bool has_sh = p.sh_gate != nullptr;

  if ((int)blockIdx.x >= p.n_router_blocks) {       // shared expert gate/up
    const int i0 = ((int)blockIdx.x - p.n_router_blocks) * kPairsPerBlock + wid * kPairsPerWave;
    if (i0 < p.Is) up_pairs<MAXC>(p.sh_gate, p.sh_up, i0, p.Is, p.H, xf, lane, p.sact_ws);
    return;
  }

  // Router rows: E logits (unless supplied) then the shared-gate logit at index E.
  const int n_lrows = p.logits_in ? 0 : p.E;
  const int n_rows = n_lrows + (has_sh ? 1 : 0);
  const int row = (int)blockIdx.x * 4 + wid;
  if (row < n_rows) {
    const uint16_t* rp[1] = {row < n_lrows ? p.router_w + (size_t)row * p.H : p.sh_gate_w};
    float d[1];
    wave_dots<MAXC, 1>(rp, xf, p.H, lane, d);
    if (lane == 0) p.logits_ws[row < n_lrows ? row : p.E] = d[0];
  }
  // Last-arriving router block finishes the routing (release/acquire at agent scope).
  __shared__ int s_last;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(p.status + kStatusRouterDone, 1u, __ATOMIC_ACQ_REL,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == (unsigned)p.n_router_blocks - 1u);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (wid == 0) {
    TopkOut o;
    o.ids32 = p.ids_ws;
    o.wf = p.w_ws;
    o.ids64 = p.ids_out;
    o.wb = p.w_out;
    o.heat = p.heat;
    const float* src = p.logits_in ? p.logits_in : p.logits_ws;
    if (p.E <= 256)
      wave_topk<4>(src, p.logits_in == nullptr, p.E, p.k, lane, o);
    else
      wave_topk<16>(src, p.logits_in == nullptr, p.E, p.k, lane, o);
  } else if (wid == 1 && p.logits_out) {
    for (int e = lane; e < p.E; e += 64)
      p.logits_out[e] = p.logits_in ? p.logits_in[e]
                                    : __hip_atomic_load(p.logits_ws + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else if (wid == 2 && lane == 0) {
    if (has_sh) {
      const float z = __hip_atomic_load(p.logits_ws + p.E, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      p.gs_ws[0] = rbf16(sigmoid_f32(rbf16(z)));
    }
    __hip_atomic_store(p.status + kStatusRouterDone, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------- B
template <int MAXC>
__global__ __launch_bounds__(256) void k_decode_b(DecodeParams p) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int n_up = p.k * p.n_up_blocks_per_expert;
  if ((int)blockIdx.x < n_up) {                      // routed gate/up for slot j
    const int j = (int)blockIdx.x / p.n_up_blocks_per_expert;
    const int i0 = ((int)blockIdx.x % p.n_up_blocks_per_expert) * kPairsPerBlock + wid * kPairsPerWave;
    int e;
    if (!slot_expert(p, j, e) || i0 >= p.I) return;
    XFrag<MAXC> xf;
    load_xfrag<MAXC>(xf, p.x, p.H, lane);
    const uint16_t* gu = reinterpret_cast<const uint16_t*>(p.table[2 * e]);
    up_pairs<MAXC>(gu, gu + (size_t)p.I * p.H, i0, p.I, p.H, xf, lane, p.act_ws + (size_t)j * p.I);
    return;
  }
  // shared down rows, scaled by the sigmoid gate
  const int h0 = ((int)blockIdx.x - n_up) * kDownRowsPerBlock + wid * kDownRowsPerWave;
  if (h0 >= p.H) return;
  XFrag<MAXC> af;
  load_xfrag<MAXC>(af, p.sact_ws, p.Is, lane);
  const uint16_t* rows[kDownRowsPerWave];
#pragma unroll
  for (int r = 0; r < kDownRowsPerWave; ++r) rows[r] = p.sh_down + (size_t)min(h0 + r, p.H - 1) * p.Is;
  float d[kDownRowsPerWave];
  wave_dots<MAXC, kDownRowsPerWave>(rows, af, p.Is, lane, d);
  if (lane == 0) {
    const float g = p.gs_ws[0];
#pragma unroll
    for (int r = 0; r < kDownRowsPerWave; ++r)
      if (h0 + r < p.H) p.sh_ws[h0 + r] = f32_to_bf16(g * rbf16(d[r]));
  }
}

// ---------------------------------------------------------------- C
// One output row per wave; the k expert rows are loaded KB at a time.
template <int MAXC, int KB>
__global__ __launch_bounds__(256) void k_decode_c(DecodeParams p) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int h = (int)blockIdx.x * 4 + wid;
  if (h >= p.H) return;
  float acc = 0.f;
  for (int j0 = 0; j0 < p.k; j0 += KB) {
    u32x4 w[KB][MAXC], a[KB][MAXC];
    bool ok[KB];
#pragma unroll
    for (int b = 0; b < KB; ++b) {
      int e = 0;
      ok[b] = (j0 + b < p.k) && slot_expert(p, j0 + b, e);
      const uint16_t* wrow = ok[b] ? reinterpret_cast<const uint16_t*>(p.table[2 * e + 1]) + (size_t)h * p.I : nullptr;
      const uint16_t* arow = p.act_ws + (size_t)(j0 + b) * p.I;
#pragma unroll
      for (int c = 0; c < MAXC; ++c) {
        const int col = c * 512 + lane * 8;
        const bool in = ok[b] && col < p.I;
        w[b][c] = in ? ld_stream(wrow + col) : u32x4{0u, 0u, 0u, 0u};
        a[b][c] = in ? ld16(arow + col) : u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int b = 0; b < KB; ++b) {
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < MAXC; ++c) s = dot8bb(w[b][c], a[b][c], s);
      const float d = rbf16(wave_sum(s));
      if (ok[b]) acc = rbf16(acc + rbf16(slot_weight(p, j0 + b) * d));
    }
  }
  if (p.sh_gate) acc = rbf16(acc + bf16_to_f32(p.sh_ws[h]));
  if (lane == 0) p.out[h] = f32_to_bf16(acc);
}

static int pick_maxc(int nc) { return nc <= 2 ? 2 : nc <= 4 ? 4 : nc <= 6 ? 6 : 8; }

template <int MAXC>
static void launch_bc(const DecodeParams& p, bool run_b, hipStream_t s) {
  if (run_b) {
    const int nb = p.k * p.n_up_blocks_per_expert + p.n_shared_down_blocks;
    hipLaunchKernelGGL(k_decode_b<MAXC>, dim3(nb), dim3(256), 0, s, p);
  }
}

int decode_launch(DecodeParams& p, bool run_router, hipStream_t s) {
  const int ncH = (p.H + 511) / 512, ncI = (p.I + 511) / 512, ncS = (p.Is + 511) / 512;
  const bool has_sh = p.sh_gate != nullptr;
  p.n_up_blocks_per_expert = (p.I + kPairsPerBlock - 1) / kPairsPerBlock;
  p.n_shared_down_blocks = has_sh ? (p.H + kDownRowsPerBlock - 1) / kDownRowsPerBlock : 0;
  p.n_shared_up_blocks = has_sh ? (p.Is + kPairsPerBlock - 1) / kPairsPerBlock : 0;
  if (run_router) {
    const int n_rows = (p.logits_in ? 0 : p.E) + (has_sh ? 1 : 0);
    p.n_router_blocks = n_rows > 0 ? (n_rows + 3) / 4 : 1;
    const dim3 ga(p.n_router_blocks + p.n_shared_up_blocks);
    switch (pick_maxc(ncH)) {
      case 2: hipLaunchKernelGGL(k_decode_a<2>, ga, dim3(256), 0, s, p); break;
      case 4: hipLaunchKernelGGL(k_decode_a<4>, ga, dim3(256), 0, s, p); break;
      case 6: hipLaunchKernelGGL(k_decode_a<6>, ga, dim3(256), 0, s, p); break;
      default: hipLaunchKernelGGL(k_decode_a<8>, ga, dim3(256), 0, s, p); break;
    }
  }
  switch (pick_maxc(ncH > ncS ? ncH : ncS)) {
    case 2: launch_bc<2>(p, true, s); break;
    case 4: launch_bc<4>(p, true, s); break;
    case 6: launch_bc<6>(p, true, s); break;
    default: launch_bc<8>(p, true, s); break;
  }
  const dim3 gc((p.H + 3) / 4);
  switch (pick_maxc(ncI)) {
    case 2: hipLaunchKernelGGL((k_decode_c<2, 8>), gc, dim3(256), 0, s, p); break;
    case 4: hipLaunchKernelGGL((k_decode_c<4, 4>), gc, dim3(256), 0, s, p); break;
    case 6: hipLaunchKernelGGL((k_decode_c<6, 2>), gc, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL((k_decode_c<8, 2>), gc, dim3(256), 0, s, p); break;
  }
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

}  // namespace tmoe

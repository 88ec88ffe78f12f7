// Prefill (T > 1) MoE layer: dispatch, MFMA grouped GEMMs, expert-ascending combine.
//
//   dispatch  histogram + exclusive scan (1 block), stable per-expert compaction
//             (1 block per expert) -> offsets, perm (expert, slot, token order), inv,
//             and the grouped-GEMM tile schedule.      tarfa/engine/fused_int4.py:228-229, 241
//   up GEMM   per group: [rows x H] . [H x 2I] on v_mfma_f32_16x16x32_bf16, epilogue
//             act = bf16(bf16(silu(bf16 g)) * bf16 u)    fused_int4.py:242-243
//   down GEMM per group: [rows x I] . [I x H], epilogue ch = bf16(bf16(d) * w[t, slot])
//             (shared group: sh = bf16(gs[t] * bf16(d)))  fused_int4.py:243
//   combine   per token, its k rows of ch added in ascending expert id with a bf16
//             rounding after each add, then + sh          fused_int4.py:244 (index_add_),
//                                                          transformers/.../modeling_qwen3_5_moe.py:796
// The shared expert is one more group (id E) whose rows are all T tokens in order.
#include "tmoe_gemv.h"
#include "tmoe_ws.h"

namespace tmoe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int kBM = 160;        // rows per M-chunk: a whole group in one block up to 160 rows
constexpr int kAS = kBM / 32;   // A rows staged per thread (rows tid/8 + 32 i)
constexpr int kBK = 64;         // K per LDS stage
constexpr int kLdsStride = 72;  // bf16 per LDS row (64 + 8 pad: spreads rows over banks)
constexpr int kRing = 3;        // K stages of A and of the weights requested ahead of the multiply
                                // (3 keeps a wave within 256 registers: two blocks per CU)

__device__ __forceinline__ int load_id(const int32_t* ids32, const int64_t* ids64, size_t i) {
  return ids32 ? ids32[i] : (int)ids64[i];
}

// ---------------------------------------------------------------- shared gate
template <int MAXC>
__global__ __launch_bounds__(256) void k_shared_gate(const uint16_t* __restrict__ x, const uint16_t* __restrict__ wsg,
                                                     int T, int H, float* __restrict__ gs) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  XFrag<MAXC> xf;
  load_xfrag<MAXC>(xf, x + (size_t)t * H, H, lane);
  const uint16_t* rows[1] = {wsg};
  float d[1];
  wave_dots<MAXC, 1>(rows, xf, H, lane, d);
  if (lane == 0) gs[t] = rbf16(sigmoid_f32(rbf16(d[0])));
}

int launch_shared_gate(const uint16_t* x, const uint16_t* w_sg, int T, int H, float* gs, hipStream_t s) {
  const int nc = (H + 511) / 512;
  const dim3 g((T + 3) / 4), b(256);
  switch (nc <= 2 ? 2 : nc <= 4 ? 4 : nc <= 6 ? 6 : 8) {
    case 2: hipLaunchKernelGGL(k_shared_gate<2>, g, b, 0, s, x, w_sg, T, H, gs); break;
    case 4: hipLaunchKernelGGL(k_shared_gate<4>, g, b, 0, s, x, w_sg, T, H, gs); break;
    case 6: hipLaunchKernelGGL(k_shared_gate<6>, g, b, 0, s, x, w_sg, T, H, gs); break;
    default: hipLaunchKernelGGL(k_shared_gate<8>, g, b, 0, s, x, w_sg, T, H, gs); break;
  }
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

// ---------------------------------------------------------------- dispatch
// One block of 1024 threads: per-expert counts, offsets, M-chunk schedule, inv := -1.
__global__ __launch_bounds__(1024) void k_dispatch_count(const int32_t* ids32, const int64_t* ids64, int T, int k,
                                                         int E, int shared_rows, int32_t* offsets,
                                                         int32_t* tile_start, int32_t* inv, uint32_t* status) {
  __shared__ int cnt[1024];
  const int tid = threadIdx.x;
  for (int e = tid; e < 1024; e += 1024) cnt[e] = 0;
  __syncthreads();
  const int n = T * k;
  bool bad = false;
  for (int j = tid; j < n; j += 1024) {
    const int e = load_id(ids32, ids64, j);
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    else if (e != E) bad = true;
    inv[j] = -1;
  }
  if (bad && status) atomicOr(status + kStatusError, 1u);
  __syncthreads();
  // Inclusive Hillis-Steele scans of counts and M-chunks (groups 0..E-1, then the shared group).
  const int c = tid < E ? cnt[tid] : 0;
  int ch = tid < E ? (c + kBM - 1) / kBM : (tid == E ? (shared_rows + kBM - 1) / kBM : 0);
  __shared__ int sc[1024], sk[1025];
  sc[tid] = c;
  sk[tid] = ch;
  if (tid == 0) sk[1024] = 0;
  __syncthreads();
  for (int d = 1; d < 1024; d <<= 1) {
    const int a = tid >= d ? sc[tid - d] : 0;
    const int b = tid >= d ? sk[tid - d] : 0;
    __syncthreads();
    sc[tid] += a;
    sk[tid] += b;
    __syncthreads();
  }
  if (tid < E) offsets[tid + 1] = sc[tid];
  if (tid == 0) { offsets[0] = 0; tile_start[0] = 0; }
  if (tid <= E) tile_start[tid + 1] = sk[tid];
}

// One block per expert: stable compaction of the slot-major traversal j = slot*T + t.
__global__ __launch_bounds__(1024) void k_dispatch_scatter(const int32_t* ids32, const int64_t* ids64, int T, int k,
                                                           const int32_t* __restrict__ offsets, int32_t* perm,
                                                           int32_t* inv) {
  __shared__ int wave_tot[16];
  const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int n = T * k;
  int running = offsets[e];
  for (int j0 = 0; j0 < n; j0 += 1024) {
    const int j = j0 + tid;
    int slot = 0, t = 0;
    bool match = false;
    if (j < n) {
      slot = j / T;
      t = j - slot * T;
      match = load_id(ids32, ids64, (size_t)t * k + slot) == e;
    }
    const uint64_t mask = __ballot(match);
    const int before = __popcll(mask & ((1ull << lane) - 1ull));
    if (lane == 0) wave_tot[wid] = __popcll(mask);
    __syncthreads();
    int wofs = 0, total = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      const int v = wave_tot[w];
      wofs += w < wid ? v : 0;
      total += v;
    }
    if (match) {
      const int r = running + wofs + before;
      perm[r] = t * k + slot;
      inv[(size_t)t * k + slot] = r;
    }
    running += total;
    __syncthreads();
  }
}

// ---------------------------------------------------------------- grouped GEMM
struct GemmParams {
  const uint16_t* a;         // up: x [T, H]; down: act [(T*k + T), I]
  int K;                     // reduction length (row stride of A and of the weights)
  int gather;                // 1: routed A row r is x[perm[r] / k] (up); 0: A row r is a[r] (down)
  const int32_t* offsets;    // [E + 1]
  const int32_t* perm;       // [T * k]
  const int32_t* tile_start; // [n_groups + 1] cumulative M-chunks
  int T, E, k, n_groups, n_ntiles, up, N, I;
  int group_lo, group_hi;    // groups [group_lo, group_hi) of this launch
  const uint64_t* table;     // [E][2] bf16; int4: [E][4] (packed, scales) x (gate_up, down)
  const uint16_t* shw0;      // shared: gate_proj (up) / down_proj (down)
  const uint16_t* shw1;      // shared: up_proj (up)
  int shared_row0;           // first act row of the shared group (T * k)
  uint16_t* out;             // up: act; down: ch [T*k, H]
  uint16_t* out_sh;          // down: sh [T, H]
  const float* wf;           // routing weights by assignment t*k + slot (fp32 holding bf16) ...
  const uint16_t* wb;        // ... or bf16
  const float* gs;           // [T] shared gate
};

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// One MFMA B fragment from int4: the 8 weights of 4 packed bytes (byte b = k 2b low
// nibble, 2b + 1 high nibble), dequantised as bf16((n - 8) * s) -- the reference's
// `dequant_int4` then bf16 `F.linear` (tarfa/engine/fused_int4.py:258-259).  n * s - 8 s
// is exact in fp32 (a 4-bit times an 8-bit significand), so one RNE to bf16 reproduces
// the dequantised matrix bit for bit (finite scales).
__device__ __forceinline__ uint32_t bf16_rne_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  return u + 0x7FFFu + ((u >> 16) & 1u);     // bf16 in the high half
}
__device__ __forceinline__ u32x4 dequant_frag(uint32_t w, float s) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  const float m8 = -8.0f * s;
  uint32_t d[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const uint32_t e = bf16_rne_bits(fmaf((float)((lo >> (8 * b)) & 0xFFu), s, m8));
    const uint32_t o = bf16_rne_bits(fmaf((float)((hi >> (8 * b)) & 0xFFu), s, m8));
    d[b] = __builtin_amdgcn_perm(o, e, 0x07060302u);   // (even k low, odd k high)
  }
  return u32x4{d[0], d[1], d[2], d[3]};
}

// Block = 4 waves; tile = (up to 256 rows of one group) x (two 16-row weight sets per
// wave).  A is staged through LDS (double-buffered, one barrier per 64-wide K stage);
// weights are read once, straight into MFMA B-fragment registers, kRing stages ahead.
// The weight loads are plain, not non-temporal: a B-fragment load covers half of each of
// 16 lines (16 rows x 64 bytes) and the next k step the other half; with the
// non-temporal hint the two halves miss separately (a 2.68 GB read in this pattern
// measured 5.1 TB/s with the hint, 6.0 without, at 256 KB per CU in flight).
// RING = K stages requested ahead of the multiply; Q4: routed weights are int4 (table
// [E][4]), dequantised into the B fragments in registers (a launch covers either the
// routed groups in int4 or the shared group in bf16, never both).
template <int RING, bool Q4>
__global__ __launch_bounds__(256, 2) void k_grouped_gemm(GemmParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][kBM * kLdsStride];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;

  // Tile index, remapped so each XCD (blocks b with equal b % 8) walks a
  // contiguous range: the N-tiles of one group share that XCD's L2 copy of A.
  const int f0 = p.tile_start[p.group_lo] * p.n_ntiles;
  const int total = p.tile_start[p.group_hi] * p.n_ntiles - f0;
  const int per_xcd = (total + 7) / 8;
  const int q = (int)blockIdx.x >> 3, xcd = (int)blockIdx.x & 7;
  if (q >= per_xcd) return;
  const int f = xcd * per_xcd + q;
  if (f >= total) return;
  const int mt = (f0 + f) / p.n_ntiles, nt = (f0 + f) - mt * p.n_ntiles;
  int lo = p.group_lo, hi = p.group_hi;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (p.tile_start[mid] <= mt) lo = mid; else hi = mid;
  }
  const int g = lo;
  const bool shared = g == p.E;
  const int r0 = (mt - p.tile_start[g]) * kBM;
  const int grow0 = shared ? 0 : p.offsets[g];
  const int gcnt = shared ? p.T : p.offsets[g + 1] - grow0;
  const int m = min(kBM, gcnt - r0);
  const int K = p.K;

  // Weight row sets of this wave: rows r0w (first set) and r1w (second set) of the
  // expert's gate_up [2I, K] or down [H, K] matrix, this lane's row (lane & 15) and k
  // offset 8 (lane >> 4) within each 32-wide k step.
  int c0, r0w, r1w;
  if (p.up) {
    c0 = nt * 64 + wid * 16;
    r0w = c0;
    r1w = shared ? c0 : p.I + c0;
  } else {
    c0 = nt * 128 + wid * 32;
    r0w = c0;
    r1w = c0 + 16;
  }
  const uint16_t *b0 = nullptr, *b1 = nullptr;      // bf16 weights
  const uint8_t *q0 = nullptr, *q1 = nullptr;       // int4: packed rows (K / 2 bytes) ...
  const uint16_t *s0 = nullptr, *s1 = nullptr;      // ... and their group scales (K / 128)
  if (Q4) {
    const int part = p.up ? 0 : 2;
    const uint8_t* pk = reinterpret_cast<const uint8_t*>(p.table[4 * g + part]);
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(p.table[4 * g + part + 1]);
    const int row = lane & 15;
    q0 = pk + (size_t)(r0w + row) * (K / 2) + 4 * (lane >> 4);
    q1 = pk + (size_t)(r1w + row) * (K / 2) + 4 * (lane >> 4);
    s0 = sc + (size_t)(r0w + row) * (K / 128);
    s1 = sc + (size_t)(r1w + row) * (K / 128);
  } else {
    const uint16_t *w0, *w1;
    if (p.up) {
      if (shared) {
        w0 = p.shw0;
        w1 = p.shw1;
      } else {
        w0 = w1 = reinterpret_cast<const uint16_t*>(p.table[2 * g]);
      }
    } else {
      w0 = w1 = shared ? p.shw0 : reinterpret_cast<const uint16_t*>(p.table[2 * g + 1]);
    }
    const int bl = (lane & 15) * K + 8 * (lane >> 4);
    b0 = w0 + (size_t)r0w * K + bl;
    b1 = w1 + (size_t)r1w * K + bl;
  }

  // A rows this thread stages: rows tid/8 + 32 i, 16-byte column chunk tid % 8.  Rows past
  // the group repeat its last row, so every load is unconditional (results of those rows
  // are never written).
  const uint16_t* arow[kAS];
#pragma unroll
  for (int i = 0; i < kAS; ++i) {
    const int r = (tid >> 3) + 32 * i;
    const int rr = r0 + min(r, m - 1);
    size_t row;
    if (p.gather) row = shared ? (size_t)rr : (size_t)(p.perm[grow0 + rr] / p.k);
    else row = shared ? (size_t)(p.shared_row0 + rr) : (size_t)(grow0 + rr);
    arow[i] = p.a + row * K + (tid & 7) * 8;
  }
  const int lds_st = (tid >> 3) * kLdsStride + (tid & 7) * 8;   // + 32 * i * kLdsStride
  const int lds_ld = (lane & 15) * kLdsStride + 8 * (lane >> 4); // + sub*16*kLdsStride + ks*32

  constexpr int kSubs = kBM / 16;
  f32x4 acc[kSubs][2];
#pragma unroll
  for (int s = 0; s < kSubs; ++s) acc[s][0] = acc[s][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Software pipeline over K stages of 64: A rows for stages s + 1 .. s + RING and weight
  // fragments for stages s .. s + RING - 1 are in flight while stage s multiplies.  An A
  // stage waits in registers until its LDS buffer frees (double-buffered); weights go
  // straight from registers into the MFMA.  Ring slots are static (the loop is unrolled
  // by RING).
  u32x4 areg[RING][kAS], breg[RING][2][2];
  uint32_t qreg[RING][2][2], sreg[RING][2];           // int4: packed words and scales in flight
  const int nk = K / kBK;
  auto load_a = [&](int slot, int st) {
    const int k0 = st * kBK;
#pragma unroll
    for (int i = 0; i < kAS; ++i) areg[slot][i] = ld16(arow[i] + k0);
  };
  auto load_b = [&](int slot, int st) {
    const int k0 = st * kBK;
    if constexpr (Q4) {
      // A 64-wide stage lies inside one 128-column scale group.
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        qreg[slot][ks][0] = *(const __attribute__((address_space(1))) uint32_t*)(q0 + (k0 + 32 * ks) / 2);
        qreg[slot][ks][1] = *(const __attribute__((address_space(1))) uint32_t*)(q1 + (k0 + 32 * ks) / 2);
      }
      sreg[slot][0] = s0[k0 / 128];
      sreg[slot][1] = s1[k0 / 128];
    } else {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        breg[slot][ks][0] = ld16(b0 + k0 + 32 * ks);
        breg[slot][ks][1] = ld16(b1 + k0 + 32 * ks);
      }
    }
  };
  auto store_a = [&](int buf, int slot) {
#pragma unroll
    for (int i = 0; i < kAS; ++i)
      *reinterpret_cast<u32x4*>(&lds[buf][lds_st + 32 * i * kLdsStride]) = areg[slot][i];
  };
  // All kSubs 16-row sub-tiles every stage, straight-line: the A fragments of a 32-wide k
  // step are read from LDS before their MFMAs issue (one LDS round trip per k step), and
  // the accumulators keep one register assignment.  Sub-tiles past the group's rows
  // multiply repeated rows whose results are never written; at ~128 rows per group that
  // is a quarter more MFMA work, well under the time the weight stream takes.
  auto multiply = [&](int buf, int slot) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8_t bg, bu;
      if constexpr (Q4) {
        bg = as_bf16x8(dequant_frag(qreg[slot][ks][0], bf16_to_f32((uint16_t)sreg[slot][0])));
        bu = as_bf16x8(dequant_frag(qreg[slot][ks][1], bf16_to_f32((uint16_t)sreg[slot][1])));
      } else {
        bg = as_bf16x8(breg[slot][ks][0]);
        bu = as_bf16x8(breg[slot][ks][1]);
      }
      u32x4 av[kSubs];
#pragma unroll
      for (int sub = 0; sub < kSubs; ++sub)
        av[sub] = *reinterpret_cast<const u32x4*>(&lds[buf][lds_ld + sub * 16 * kLdsStride + ks * 32]);
#pragma unroll
      for (int sub = 0; sub < kSubs; ++sub) {
        const bf16x8_t a = as_bf16x8(av[sub]);
        acc[sub][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bg, acc[sub][0], 0, 0, 0);
        acc[sub][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bu, acc[sub][1], 0, 0, 0);
      }
    }
  };
  // Every refill is unconditional: a stage index past the end is clamped to the last
  // stage (a repeat of addresses just read, served by the L2), so the compiler's
  // in-order count of outstanding loads stays exact and each wait covers one stage;
  // only the multiply (LDS reads and MFMA, no global loads) sits behind a branch.
  const int last = nk - 1;
  // Prologue: stages 0 .. RING - 1 requested, stage 0 staged in LDS, its register slot
  // refilled with stage RING.
#pragma unroll
  for (int st = 0; st < RING; ++st) {
    load_a(st, min(st, last));
    load_b(st, min(st, last));
  }
  store_a(0, 0);
  load_a(0, min(RING, last));
  __syncthreads();
  // Stage st (ring slot u = st % RING): stage st + 1's A to the other LDS buffer (last
  // read before the previous barrier), its register slot refilled with stage
  // st + 1 + RING; multiply stage st; refill its weight slot with stage st + RING.
  for (int st0 = 0; st0 < nk; st0 += RING) {
#pragma unroll
    for (int u = 0; u < RING; ++u) {
      const int st = st0 + u;
      store_a((st + 1) & 1, (u + 1) % RING);
      load_a((u + 1) % RING, min(st + 1 + RING, last));
      if (st < nk) multiply(st & 1, u);
      load_b(u, min(st + RING, last));
      __syncthreads();
    }
  }

  // Epilogue.  C fragment: lane l holds rows 4*(l/16) + i, column l % 16.
  const int col = c0 + (lane & 15);
  const int rl = 4 * (lane >> 4);
  if (p.up) {
    uint16_t* o = p.out + (size_t)(shared ? p.shared_row0 + r0 : grow0 + r0) * p.N + col;
#pragma unroll
    for (int sub = 0; sub < kSubs; ++sub)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = sub * 16 + rl + i;
        const uint16_t v = f32_to_bf16(swiglu_bf16(rbf16(acc[sub][0][i]), rbf16(acc[sub][1][i])));
        if (row < m) o[(size_t)row * p.N] = v;
      }
  } else if (shared) {
    uint16_t* o = p.out_sh + (size_t)r0 * p.N + col;
#pragma unroll
    for (int sub = 0; sub < kSubs; ++sub)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = sub * 16 + rl + i;
        const float gv = p.gs[r0 + min(row, m - 1)];
        const uint16_t v0 = f32_to_bf16(gv * rbf16(acc[sub][0][i])), v1 = f32_to_bf16(gv * rbf16(acc[sub][1][i]));
        if (row < m) { o[(size_t)row * p.N] = v0; o[(size_t)row * p.N + 16] = v1; }
      }
  } else {
    uint16_t* o = p.out + (size_t)(grow0 + r0) * p.N + col;
    const int32_t* pr = p.perm + grow0 + r0;
#pragma unroll
    for (int sub = 0; sub < kSubs; ++sub)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = sub * 16 + rl + i;
        const int a = pr[min(row, m - 1)];
        const float w = p.wf ? p.wf[a] : bf16_to_f32(p.wb[a]);
        const uint16_t v0 = f32_to_bf16(rbf16(acc[sub][0][i]) * w), v1 = f32_to_bf16(rbf16(acc[sub][1][i]) * w);
        if (row < m) { o[(size_t)row * p.N] = v0; o[(size_t)row * p.N + 16] = v1; }
      }
  }
}

// ---------------------------------------------------------------- combine
// One wave per token; lane owns 8 columns per 512-column chunk.
template <int MAXC>
__global__ __launch_bounds__(256) void k_combine(const int32_t* ids32, const int64_t* ids64,
                                                 const int32_t* __restrict__ inv, const uint16_t* __restrict__ ch,
                                                 const uint16_t* __restrict__ sh, int T, int H, int E, int k,
                                                 uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  // The token's valid (expert, slot) entries sorted ascending: index_add_ order.
  int ke[16], kr[16], n = 0;
  for (int s = 0; s < k; ++s) {
    const int e = load_id(ids32, ids64, (size_t)t * k + s);
    const int r = inv[(size_t)t * k + s];
    if (e < 0 || e >= E || r < 0) continue;
    int pos = n++;
    while (pos > 0 && ke[pos - 1] > e) { ke[pos] = ke[pos - 1]; kr[pos] = kr[pos - 1]; --pos; }
    ke[pos] = e;
    kr[pos] = r;
  }
  float acc[MAXC][8];
#pragma unroll
  for (int c = 0; c < MAXC; ++c)
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[c][q] = 0.f;
  for (int j = 0; j < n; ++j) {
    const uint16_t* row = ch + (size_t)kr[j] * H;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int col = c * 512 + lane * 8;
      if (col < H) {
        const u32x4 v = ld16(row + col);
        acc[c][0] = rbf16(acc[c][0] + bf16_lo(v.x)); acc[c][1] = rbf16(acc[c][1] + bf16_hi(v.x));
        acc[c][2] = rbf16(acc[c][2] + bf16_lo(v.y)); acc[c][3] = rbf16(acc[c][3] + bf16_hi(v.y));
        acc[c][4] = rbf16(acc[c][4] + bf16_lo(v.z)); acc[c][5] = rbf16(acc[c][5] + bf16_hi(v.z));
        acc[c][6] = rbf16(acc[c][6] + bf16_lo(v.w)); acc[c][7] = rbf16(acc[c][7] + bf16_hi(v.w));
      }
    }
  }
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int col = c * 512 + lane * 8;
    if (col >= H) continue;
    if (sh) {
      const u32x4 v = ld16(sh + (size_t)t * H + col);
      acc[c][0] = rbf16(acc[c][0] + bf16_lo(v.x)); acc[c][1] = rbf16(acc[c][1] + bf16_hi(v.x));
      acc[c][2] = rbf16(acc[c][2] + bf16_lo(v.y)); acc[c][3] = rbf16(acc[c][3] + bf16_hi(v.y));
      acc[c][4] = rbf16(acc[c][4] + bf16_lo(v.z)); acc[c][5] = rbf16(acc[c][5] + bf16_hi(v.z));
      acc[c][6] = rbf16(acc[c][6] + bf16_lo(v.w)); acc[c][7] = rbf16(acc[c][7] + bf16_hi(v.w));
    }
    u32x4 o;
    o.x = f32_to_bf16(acc[c][0]) | ((uint32_t)f32_to_bf16(acc[c][1]) << 16);
    o.y = f32_to_bf16(acc[c][2]) | ((uint32_t)f32_to_bf16(acc[c][3]) << 16);
    o.z = f32_to_bf16(acc[c][4]) | ((uint32_t)f32_to_bf16(acc[c][5]) << 16);
    o.w = f32_to_bf16(acc[c][6]) | ((uint32_t)f32_to_bf16(acc[c][7]) << 16);
    *reinterpret_cast<u32x4*>(out + (size_t)t * H + col) = o;
  }
}

// ---------------------------------------------------------------- driver
int dispatch_launch(const int32_t* ids32, const int64_t* ids64, int T, int k, int E, int shared_rows,
                    int32_t* offsets, int32_t* perm, int32_t* inv, int32_t* tile_start, uint32_t* status,
                    hipStream_t s) {
  hipLaunchKernelGGL(k_dispatch_count, dim3(1), dim3(1024), 0, s, ids32, ids64, T, k, E, shared_rows, offsets,
                     tile_start, inv, status);
  hipLaunchKernelGGL(k_dispatch_scatter, dim3(E), dim3(1024), 0, s, ids32, ids64, T, k, offsets, perm, inv);
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

int prefill_launch(const uint16_t* x, int T, const int32_t* ids32, const int64_t* ids64, const float* wf,
                   const uint16_t* wb, const uint64_t* table, const uint16_t* sh_gate, const uint16_t* sh_up,
                   const uint16_t* sh_down, const float* gs, int H, int E, int I, int k, int Is, uint16_t* out,
                   void* ws, hipStream_t s, bool q4) {
  const bool has_sh = sh_gate != nullptr;
  if (H % 128 || I % 64 || E > 1023 || (has_sh && Is != I)) return TMOE_ERR_SHAPE;
  if (q4 && I % 128) return TMOE_ERR_SHAPE;   // int4: every 64-wide K stage inside one 128-column group
  const Ws L = ws_layout(T, H, E, I, k, Is);
  int32_t* offsets = ws_ptr<int32_t>(ws, L.offsets);
  int32_t* perm = ws_ptr<int32_t>(ws, L.perm);
  int32_t* inv = ws_ptr<int32_t>(ws, L.inv);
  int32_t* tile_start = ws_ptr<int32_t>(ws, L.scratch);
  uint32_t* status = ws_ptr<uint32_t>(ws, L.status);
  uint16_t* act = ws_ptr<uint16_t>(ws, L.act);
  uint16_t* ch = ws_ptr<uint16_t>(ws, L.ch);
  uint16_t* sh = ws_ptr<uint16_t>(ws, L.sh);
  if (int st = dispatch_launch(ids32, ids64, T, k, E, has_sh ? T : 0, offsets, perm, inv, tile_start, status, s))
    return st;

  const int n_groups = has_sh ? E + 1 : E;
  const long mbound = (long)T * k / kBM + (long)(E < T * k ? E : T * k) + (has_sh ? (T + kBM - 1) / kBM : 0) + 1;
  const long mshared = (T + kBM - 1) / kBM;

  // One GEMM over groups [lo, hi): bf16 weights, or int4 routed weights (the shared
  // group, always bf16, then gets a launch of its own).
  auto gemm = [&](GemmParams g, int lo, int hi, bool routed_q4, long mchunks) {
    g.group_lo = lo;
    g.group_hi = hi;
    const long grid = (mchunks * g.n_ntiles + 7) / 8 * 8;
    if (routed_q4)
      hipLaunchKernelGGL((k_grouped_gemm<kRing, true>), dim3((unsigned)grid), dim3(256), 0, s, g);
    else
      hipLaunchKernelGGL((k_grouped_gemm<kRing, false>), dim3((unsigned)grid), dim3(256), 0, s, g);
  };
  GemmParams up{};
  up.a = x; up.K = H; up.gather = 1; up.offsets = offsets; up.perm = perm; up.tile_start = tile_start;
  up.T = T; up.E = E; up.k = k; up.n_groups = n_groups; up.n_ntiles = I / 64; up.up = 1; up.N = I; up.I = I;
  up.table = table; up.shw0 = sh_gate; up.shw1 = sh_up; up.shared_row0 = T * k; up.out = act;
  GemmParams dn = up;
  dn.a = act; dn.K = I; dn.gather = 0; dn.n_ntiles = H / 128; dn.up = 0; dn.N = H;
  dn.shw0 = sh_down; dn.shw1 = nullptr; dn.out = ch; dn.out_sh = sh; dn.wf = wf; dn.wb = wb; dn.gs = gs;
  if (q4) {
    gemm(up, 0, E, true, mbound);
    if (has_sh) gemm(up, E, E + 1, false, mshared);
    gemm(dn, 0, E, true, mbound);
    if (has_sh) gemm(dn, E, E + 1, false, mshared);
  } else {
    gemm(up, 0, n_groups, false, mbound);
    gemm(dn, 0, n_groups, false, mbound);
  }

  const int nc = (H + 511) / 512;
  const dim3 gc((T + 3) / 4), bc(256);
  const uint16_t* shp = has_sh ? sh : nullptr;
  switch (nc <= 2 ? 2 : nc <= 4 ? 4 : nc <= 6 ? 6 : 8) {
    case 2: hipLaunchKernelGGL(k_combine<2>, gc, bc, 0, s, ids32, ids64, inv, ch, shp, T, H, E, k, out); break;
    case 4: hipLaunchKernelGGL(k_combine<4>, gc, bc, 0, s, ids32, ids64, inv, ch, shp, T, H, E, k, out); break;
    case 6: hipLaunchKernelGGL(k_combine<6>, gc, bc, 0, s, ids32, ids64, inv, ch, shp, T, H, E, k, out); break;
    default: hipLaunchKernelGGL(k_combine<8>, gc, bc, 0, s, ids32, ids64, inv, ch, shp, T, H, E, k, out); break;
  }
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

}  // namespace tmoe

extern "C" int tmoe_dispatch(const int64_t* ids, int T, int k, int E, int32_t* offsets, int32_t* perm, int32_t* inv,
                             void* workspace, size_t ws_bytes, void* stream) {
  using namespace tmoe;
  if (T < 1 || k < 1 || k > 16 || E < 1 || E > 1023) return TMOE_ERR_SHAPE;
  if (!ids || !offsets || !perm || !inv || !workspace) return TMOE_ERR_NULL;
  const Ws L = ws_layout(T, 8, E, 8, k, 0);
  if (ws_bytes < L.scratch + sizeof(int32_t) * (size_t)(E + 64)) return TMOE_ERR_WORKSPACE;
  return dispatch_launch(nullptr, ids, T, k, E, 0, offsets, perm, inv, ws_ptr<int32_t>(workspace, L.scratch),
                         ws_ptr<uint32_t>(workspace, L.status), (hipStream_t)stream);
}

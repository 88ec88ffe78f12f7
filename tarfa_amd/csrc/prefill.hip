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
#include <stdlib.h>
#include <string.h>
#include <type_traits>
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
// Ids 4q .. 4q + 3 with 16-byte loads (the pointer 16-byte aligned).
__device__ __forceinline__ int4 load_id4(const int32_t* ids32, const int64_t* ids64, size_t q) {
  if (ids32) return *reinterpret_cast<const int4*>(ids32 + 4 * q);
  const longlong2 a = *reinterpret_cast<const longlong2*>(ids64 + 4 * q);
  const longlong2 b = *reinterpret_cast<const longlong2*>(ids64 + 4 * q + 2);
  return int4{(int)a.x, (int)a.y, (int)b.x, (int)b.y};
}
__device__ __forceinline__ bool ids_aligned(const int32_t* ids32, const int64_t* ids64) {
  return ((ids32 ? (uintptr_t)ids32 : (uintptr_t)ids64) & 15u) == 0;
}

// ---------------------------------------------------------------- dispatch
// One block of 1024 threads: per-expert counts, offsets, M-chunk schedule, inv := -1, and
// (desc non-null) one descriptor per M-chunk: {group, rows, first row in group order, 0}.
__global__ __launch_bounds__(1024) void k_dispatch_count(const int32_t* ids32, const int64_t* ids64, int T, int k,
                                                         int E, int shared_rows, int32_t* offsets,
                                                         int32_t* tile_start, int32_t* inv, uint32_t* err,
                                                         int4* desc) {
  __shared__ int cnt[1024];
  const int tid = threadIdx.x;
  for (int e = tid; e < 1024; e += 1024) cnt[e] = 0;
  __syncthreads();
  const int n = T * k;
  bool bad = false;
  auto take = [&](int e) {
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    else if (e != E) bad = true;
  };
  // Four ids per 16-byte load, 8 loads in flight per thread (T=4096, k=8: one round trip), when
  // the ids and inv are 16-byte aligned; the remainder one at a time.
  const int nq = ids_aligned(ids32, ids64) && ((uintptr_t)inv & 15u) == 0 ? n / 4 : 0;
  for (int q0 = tid; q0 < nq; q0 += 8 * 1024) {
    int4 ev[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) ev[u] = q0 + u * 1024 < nq ? load_id4(ids32, ids64, q0 + u * 1024) : int4{E, E, E, E};
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int q = q0 + u * 1024;
      if (q >= nq) continue;
      take(ev[u].x);
      take(ev[u].y);
      take(ev[u].z);
      take(ev[u].w);
      reinterpret_cast<int4*>(inv)[q] = int4{-1, -1, -1, -1};
    }
  }
  for (int j = 4 * nq + tid; j < n; j += 1024) {
    take(load_id(ids32, ids64, j));
    inv[j] = -1;
  }
  if (bad && err) atomicOr(err, 1u);
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
  if (!desc) return;
  // M-chunk mt of group g (sk[g - 1] <= mt < sk[g]): rows r0 = (mt - sk[g - 1]) kBM onwards.
  const int n_groups = shared_rows > 0 ? E + 1 : E;
  const int n_chunks = sk[n_groups - 1];
  for (int mt = tid; mt < n_chunks; mt += 1024) {
    int lo = 0, hi = n_groups - 1;              // the first g with sk[g] > mt
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (sk[mid] > mt) hi = mid; else lo = mid + 1;
    }
    const int g = lo;
    const int r0 = (mt - (g ? sk[g - 1] : 0)) * kBM;
    const int rows = g < E ? cnt[g] : shared_rows;
    const int first = g < E ? (g ? sc[g - 1] : 0) : 0;
    desc[mt] = int4{g, min(kBM, rows - r0), first + r0, 0};
  }
}

// One block per expert: stable compaction of the slot-major traversal j = slot*T + t.
// The block reads the ids once in memory order (i = t*k + slot, coalesced) and marks its
// expert's entries in an LDS bitmask indexed by j; thread i then owns the whole words
// [i wpt, (i + 1) wpt) of the mask: it counts their bits, one block-wide exclusive scan
// gives its first position, and it writes perm and inv for its set bits in j order.
constexpr int kScatterMaxN = 1 << 19;   // T*k up to 512 Ki entries (a 64 KB mask)
__global__ __launch_bounds__(1024) void k_dispatch_scatter(const int32_t* ids32, const int64_t* ids64, int T, int k,
                                                           const int32_t* __restrict__ offsets, int32_t* perm,
                                                           int32_t* inv) {
  __shared__ uint32_t mask[kScatterMaxN / 32];
  __shared__ int wave_tot[16];
  const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int n = T * k;
  const int nw = (n + 31) / 32;
  for (int w = tid; w < nw; w += 1024) mask[w] = 0u;
  __syncthreads();
  auto mark = [&](int i) {
    const int t = i / k, slot = i - t * k, j = slot * T + t;
    atomicOr(&mask[j >> 5], 1u << (j & 31));
  };
  // Four ids per 16-byte load, 8 loads in flight per thread, when aligned; the rest one at a time.
  const int nq = ids_aligned(ids32, ids64) ? n / 4 : 0;
  for (int q0 = tid; q0 < nq; q0 += 8 * 1024) {
    int4 ev[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) ev[u] = q0 + u * 1024 < nq ? load_id4(ids32, ids64, q0 + u * 1024) : int4{-1, -1, -1, -1};
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = 4 * (q0 + u * 1024);
      if (ev[u].x == e) mark(i);
      if (ev[u].y == e) mark(i + 1);
      if (ev[u].z == e) mark(i + 2);
      if (ev[u].w == e) mark(i + 3);
    }
  }
  for (int i = 4 * nq + tid; i < n; i += 1024)
    if (load_id(ids32, ids64, i) == e) mark(i);
  __syncthreads();
  const int wpt = (nw + 1023) / 1024;
  const int w_lo = min(nw, tid * wpt), w_hi = min(nw, w_lo + wpt);
  int c = 0;
  for (int w = w_lo; w < w_hi; ++w) c += __popc(mask[w]);
  // Block-wide exclusive scan of c: inclusive within the wave, then the waves' totals.
  int incl = c;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int v = __shfl_up(incl, d);
    if (lane >= d) incl += v;
  }
  if (lane == 63) wave_tot[wid] = incl;
  __syncthreads();
  int before = incl - c;
#pragma unroll
  for (int w = 0; w < 16; ++w) before += w < wid ? wave_tot[w] : 0;
  int r = offsets[e] + before;
  for (int w = w_lo; w < w_hi && c > 0; ++w) {
    for (uint32_t m = mask[w]; m; m &= m - 1) {
      const int j = 32 * w + __ffs(m) - 1, slot = j / T, t = j - slot * T;
      perm[r] = t * k + slot;
      inv[(size_t)t * k + slot] = r;
      ++r;
    }
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
  uint16_t* out;             // up: act; down: ch [T*k, H], each expert output unscaled
  uint16_t* out_sh;          // down: sh [T, H], the shared expert's output before its gate
  const int4* desc;          // persistent kernel: M-chunk descriptors {group, rows, first row, 0}
  uint16_t* sink;            // 16 bytes nobody reads: whole-line kernel stores of rows past a tile
};

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// One MFMA B fragment from int4: the 8 weights of 4 packed bytes (byte b = k 2b low
// nibble, 2b + 1 high nibble), dequantised as bf16((n - 8) * s) -- the reference's
// `dequant_int4` then bf16 `F.linear` (tarfa/engine/fused_int4.py:258-259).  n * s - 8 s
// is exact in fp32 (a 4-bit times an 8-bit significand), so one round-to-nearest-even to
// bf16 (v_cvt_pk_bf16_f32, two values per instruction) reproduces the dequantised matrix
// bit for bit (finite scales).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x4 dequant_frag(uint32_t w, float s) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  const float m8 = -8.0f * s;
  uint32_t d[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const float e = fmaf((float)((lo >> (8 * b)) & 0xFFu), s, m8);
    const float o = fmaf((float)((hi >> (8 * b)) & 0xFFu), s, m8);
    const bf16x2_t v = {(__bf16)e, (__bf16)o};   // (even k low, odd k high)
    d[b] = __builtin_bit_cast(uint32_t, v);
  }
  return u32x4{d[0], d[1], d[2], d[3]};
}
// A scale's 16 bits as fp32: bf16 (group scales) or fp16 (QR, per-row scales).
template <bool QR>
__device__ __forceinline__ float scale_f32(uint16_t b) {
  if constexpr (QR) return (float)__builtin_bit_cast(_Float16, b);
  else return bf16_to_f32(b);
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
// QR (with Q4): the reference's scale layout, one fp16 scale per weight row; the weight is
// then bf16((n - 8) * s) with s that row's scale (the product is exact in fp32).
template <int RING, bool Q4, bool QR = false>
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
    s0 = sc + (size_t)(r0w + row) * (QR ? 1 : K / 128);
    s1 = sc + (size_t)(r1w + row) * (QR ? 1 : K / 128);
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
      sreg[slot][0] = s0[QR ? 0 : k0 / 128];
      sreg[slot][1] = s1[QR ? 0 : k0 / 128];
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
        bg = as_bf16x8(dequant_frag(qreg[slot][ks][0], scale_f32<QR>((uint16_t)sreg[slot][0])));
        bu = as_bf16x8(dequant_frag(qreg[slot][ks][1], scale_f32<QR>((uint16_t)sreg[slot][1])));
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
  } else {
    // Down: the expert's (or the shared expert's) output, unscaled; the combine applies
    // the routing weight (or the shared gate).
    uint16_t* o = shared ? p.out_sh + (size_t)r0 * p.N + col : p.out + (size_t)(grow0 + r0) * p.N + col;
#pragma unroll
    for (int sub = 0; sub < kSubs; ++sub)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = sub * 16 + rl + i;
        const uint16_t v0 = f32_to_bf16(acc[sub][0][i]), v1 = f32_to_bf16(acc[sub][1][i]);
        if (row < m) { o[(size_t)row * p.N] = v0; o[(size_t)row * p.N + 16] = v1; }
      }
  }
}

// ---------------------------------------------------------------- grouped GEMM, persistent
// One block of 8 waves per CU, walking a list of tiles with one continuous load pipeline:
// the loads of a tile's first stages are issued during the previous tile's last stages, so
// no tile pays a pipeline fill.  Tile: kBM rows of one group x 8 waves x 32 weight rows
// (up: 16 gate rows and the matching 16 up rows per wave, 128 activation columns per
// tile; down: 32 output columns per wave, 256 per tile), K in stages of 64.
//   A (the group's rows, contiguous: the gathered token rows for up, the activations for
//   down) goes global -> LDS directly (global_load_lds_dwordx4, lane l's 16 bytes land at
//   16 l of the load's 1 KB): a load covers 8 whole rows of the stage (8 x 128 B, full
//   cache lines), lane l taking row l / 8 and 16-byte chunk (l % 8) ^ (l / 8).  Row r's
//   chunk c thus sits in LDS chunk c ^ (r % 8): the MFMA's 16-byte fragment reads (16
//   rows, one chunk) hit 8 distinct chunks per 8 lanes, conflict-free.  20 loads per
//   stage over 8 waves: each wave issues 3, the last 4 repeating loads 16..19 (the same
//   bytes to the same place), so every wave issues the same sequence.
//   B (the weights, each byte read once) goes straight into MFMA B-fragment registers
//   with plain loads, kPB stages ahead.
// Vector memory completes in issue order: the wait for weight stage s (issued kPB stages
// ahead) also covers every older load, so about kPB stages of loads (~200 KB per CU) stay
// in flight; the A ring is deeper (kPA stages) so that its waits never come first.
// Tile data (group, rows, weight pointers) is read with scalar loads from the M-chunk
// descriptors written by the dispatch.
constexpr int kPW = 8;                  // waves per block
constexpr int kPNB = 2;                 // 16-row weight blocks per wave
constexpr int kPMB = kBM / 16;          // 16-row token blocks per tile
constexpr int kPR = 8;                  // A ring slots in LDS (and the unrolled cycle)
constexpr int kPA = kPR - 1;            // A stages loaded ahead
constexpr int kPB = 4;                  // B ring slots in registers: B stages loaded ahead
constexpr int kPSlot = kBM * 8;         // u32x4 per A slot (kBM rows x 128 B = 20 KB)
constexpr int kPLoads = 3;              // A loads per wave per stage
constexpr int kPUpCols = 16 * kPW, kPDnCols = 32 * kPW;
static_assert(kBM / 8 <= kPW * kPLoads && kBM / 8 > kPW * (kPLoads - 1), "A loads cover the stage once");

// s_waitcnt vmcnt(N), as inline asm: the compiler does not see the pipeline's loads, so a
// builtin wait could look redundant to it and be dropped.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
// Scalar loads of launch-constant data (written by an earlier kernel), waited for at once.
// The address is wave-uniform; readfirstlane puts it in SGPRs for the compiler too.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ int sload1(const void* p) {
  p = uniform_ptr(p);
  int v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
  return v;
}
__device__ __forceinline__ i32x4 sload4(const void* p) {
  p = uniform_ptr(p);
  i32x4 v;
  asm volatile("s_load_dwordx4 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
  return v;
}
__device__ __forceinline__ const void* sload_ptr(const void* p) {
  p = uniform_ptr(p);
  i32x2 v;
  asm volatile("s_load_dwordx2 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
  return reinterpret_cast<const void*>(((uint64_t)(uint32_t)v.y << 32) | (uint32_t)v.x);
}

// Pipeline loads as inline asm: the compiler does not count them, so its own waits (for
// the loads it does see) can only come out stricter, and it inserts none for these; the
// kernel waits for them explicitly.  Uniform base (SGPRs) + 32-bit per-lane byte offset.
__device__ __forceinline__ u32x4 gld16(const void* sbase, uint32_t voff) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(v) : "v"(voff), "s"(sbase));
  return v;
}
__device__ __forceinline__ u32x2 gld8(const void* sbase, uint32_t voff) {
  u32x2 v;
  asm volatile("global_load_dwordx2 %0, %1, %2" : "=v"(v) : "v"(voff), "s"(sbase));
  return v;
}
__device__ __forceinline__ uint32_t gld4(const void* sbase, uint32_t voff) {
  uint32_t v;
  asm volatile("global_load_dword %0, %1, %2" : "=v"(v) : "v"(voff), "s"(sbase));
  return v;
}
__device__ __forceinline__ uint32_t gld2(const void* sbase, uint32_t voff) {
  uint32_t v;
  asm volatile("global_load_ushort %0, %1, %2" : "=v"(v) : "v"(voff), "s"(sbase));
  return v;
}
// 16 bytes per lane from global memory straight into LDS at lds + 16 lane (M0 = lds).
// Nothing else in the kernel uses M0.
__device__ __forceinline__ void gdma16(const void* sbase, uint32_t voff, const void* lds) {
  const uint32_t l = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)lds;
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(sbase), "s"(l) : "memory");
}

// 16 bytes per lane into LDS at lds + OFS (an LDS write the compiler does not reorder with
// the pipeline's asm loads and waits).
template <int OFS>
__device__ __forceinline__ void dsw16(uint32_t lds, const u32x4& v) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(lds), "v"(v), "n"(OFS) : "memory");
}

// s_waitcnt vmcnt(N) with four registers passed through it (nothing reads them before).
template <int N, typename T>
__device__ __forceinline__ void wait_vm_regs(T& a, T& b, T& c, T& d) {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(N));
}

// One wave's view of one tile (all wave-uniform).
struct PTile {
  int arow0;                // A row of the tile's first row (gather: its position in perm)
  bool gather;              // up, routed: A rows are x[perm[arow0 + r] / k]
  const uint16_t* b[kPNB];  // bf16: this wave's weight rows (row + lane's row and k offset added later)
  const uint8_t* q[kPNB];   // int4: packed rows
  const uint16_t* sc[kPNB]; // int4: scale rows
  uint16_t* o;              // first output row, this tile's first column
  int m;                    // valid rows
};

template <bool Q4, bool QR = false>
__global__ __launch_bounds__(64 * kPW, 1) void k_grouped_gemm_p(GemmParams p) {
  __shared__ u32x4 lA0[kPSlot], lA1[kPSlot], lA2[kPSlot], lA3[kPSlot], lA4[kPSlot], lA5[kPSlot], lA6[kPSlot],
      lA7[kPSlot];
  u32x4* const slots[kPR] = {lA0, lA1, lA2, lA3, lA4, lA5, lA6, lA7};
  static_assert(kPR == 8, "one LDS array per ring slot");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = p.K;
  const int cols = p.up ? kPUpCols : kPDnCols;
  // B stages in flight.  Int4: 8 (a stage is 2 KB per wave: with 4, ~1 TB/s of weights).
  constexpr int kB = Q4 ? kPR : kPB;

  // Tiles f = (M-chunk - c_lo) * n_ntiles + N-tile.  XCD x (blocks b with b % 8 == x) takes
  // the contiguous range [x per_xcd, (x + 1) per_xcd); its blocks interleave over it, so the
  // N-tiles of one group run together on one XCD and share its L2 copy of the group's rows.
  const int c_lo = sload1(p.tile_start + p.group_lo);
  const int c_hi = sload1(p.tile_start + p.group_hi);
  const int total = (c_hi - c_lo) * p.n_ntiles;
  const int nbx = (int)gridDim.x >> 3;              // blocks per XCD
  const int xcd = (int)blockIdx.x & 7, qb = (int)blockIdx.x >> 3;
  const int per_xcd = (total + 7) / 8;
  const int f0 = xcd * per_xcd + qb;
  const int f_end = min(total, (xcd + 1) * per_xcd);
  if (f0 >= f_end) return;
  const int ntile = (f_end - f0 + nbx - 1) / nbx;

  auto tile = [&](int j) {
    const int f = f0 + j * nbx;
    const int mt = c_lo + f / p.n_ntiles, nt = f % p.n_ntiles;
    const i32x4 d = sload4(p.desc + mt);
    const int g = d.x, row0 = d.z;
    const bool shared = g == p.E;
    PTile t;
    t.m = d.y;
    t.gather = p.up && !shared;
    t.arow0 = (!p.up && shared ? p.shared_row0 : 0) + row0;
    const int c0 = p.up ? nt * kPUpCols + wid * 16 : nt * kPDnCols + wid * 32;
    if (p.up) t.o = p.out + (size_t)(shared ? p.shared_row0 + row0 : row0) * p.N + nt * kPUpCols;
    else t.o = (shared ? p.out_sh : p.out) + (size_t)row0 * p.N + nt * kPDnCols;
    if constexpr (Q4) {
      const int part = p.up ? 0 : 2;
      const uint8_t* pk = reinterpret_cast<const uint8_t*>(sload_ptr(p.table + 4 * g + part));
      const uint16_t* sc = reinterpret_cast<const uint16_t*>(sload_ptr(p.table + 4 * g + part + 1));
#pragma unroll
      for (int nb = 0; nb < kPNB; ++nb) {
        const int wr = p.up ? (nb ? p.I : 0) + c0 : c0 + 16 * nb;
        t.q[nb] = pk + (size_t)wr * (K / 2);
        t.sc[nb] = sc + (size_t)wr * (QR ? 1 : K / 128);
        t.b[nb] = nullptr;
      }
    } else {
      const uint16_t *w0, *w1;
      if (shared) {
        w0 = p.shw0;
        w1 = p.up ? p.shw1 : p.shw0;
      } else {
        w0 = w1 = reinterpret_cast<const uint16_t*>(sload_ptr(p.table + 2 * g + (p.up ? 0 : 1)));
      }
#pragma unroll
      for (int nb = 0; nb < kPNB; ++nb) {
        const int wr = p.up ? ((nb && !shared) ? p.I : 0) + c0 : c0 + 16 * nb;
        t.b[nb] = (nb ? w1 : w0) + (size_t)wr * K;
        t.q[nb] = nullptr;
        t.sc[nb] = nullptr;
      }
    }
    return t;
  };

  PTile cur, nxt;   // the tile being multiplied and the one after it

  // Lane constants.  A: load j of this wave covers rows 8 x .. 8 x + 7 (x = wid + 8 j, the
  // last four repeating 16..19); B: row lane % 16 of each block, k offset 8 (lane / 16).
  // Int4: lane group g = lane / 16 loads bytes 8 g .. 8 g + 7 of its row's 32-byte stage (k
  // 16 g .. 16 g + 15) in one instruction, the first four bytes its fragment of k step 0 and
  // the last four of k step 1; its A fragments are then 16-byte chunks 2 g and 2 g + 1 of the
  // stage, the same k values (a permutation of k within the stage, applied to both operands).
  const int lrow = lane & 15, lk = 8 * (lane >> 4);
  int a_row[kPLoads];
#pragma unroll
  for (int j = 0; j < kPLoads; ++j) {
    const int x = wid + kPW * j;
    a_row[j] = 8 * (x < kBM / 8 ? x : x - kPW / 2) + (lane >> 3);
  }
  const int a_col = 8 * ((lane & 7) ^ (lane >> 3));
  const int a_ch0 = Q4 ? 2 * (lane >> 4) : lane >> 4, a_ch1 = Q4 ? 2 * (lane >> 4) + 1 : 4 + (lane >> 4);
  const int a_rd0 = lrow * 8 + (a_ch0 ^ (lrow & 7));
  const int a_rd1 = lrow * 8 + (a_ch1 ^ (lrow & 7));

  f32x4 acc[kPMB][kPNB];
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < kPMB; ++i)
#pragma unroll
      for (int nb = 0; nb < kPNB; ++nb) acc[i][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  zero_acc();

  u32x4 breg[Q4 ? 1 : kB][kPNB][2];
  uint32_t qreg[kB][kPNB][2], sreg[kB][kPNB];
  const int nk = K / kBK;   // a multiple of kPR
  // Stage st of tile cur, or (nx) stage st of tile nxt: the pointers are selected, not
  // branched on, so every path issues the same loads.
  // Addresses: a wave-uniform base (SGPRs) plus a 32-bit per-lane byte offset, the
  // global_load saddr form.  A offsets depend on the tile's row count (rows past it repeat
  // the last row) and are kept for the current and the next tile.
  const uint32_t b_off = (uint32_t)((lrow * K + lk) * 2);
  const uint32_t q_off = (uint32_t)(lrow * (K / 2) + lk);
  const uint32_t s_off = (uint32_t)(lrow * (QR ? 1 : K / 128) * 2);
  // A rows: up: x[perm[arow0 + r] / k] (routed) or x[arow0 + r] (shared); down:
  // act[arow0 + r].  Rows past the tile's count repeat its last row.  The perm entries of
  // a tile are fetched (pipeline loads, not counted by the compiler) a whole tile before
  // its offsets are formed; by then the stage waits have covered them.
  uint32_t a_off_cur[kPLoads], a_off_nxt[kPLoads];
  uint32_t pv_cur[kPLoads], pv_nxt[kPLoads];
  auto fetch_perm = [&](uint32_t* pv, const PTile& t) {
    if (!t.gather) return;
    const int32_t* pp = p.perm + t.arow0;
#pragma unroll
    for (int j = 0; j < kPLoads; ++j) pv[j] = gld4(pp, (uint32_t)(min(a_row[j], t.m - 1) * 4));
  };
  auto a_offsets = [&](uint32_t* o, uint32_t* pv, const PTile& t) {
    asm volatile("" : "+v"(pv[0]), "+v"(pv[1]), "+v"(pv[2]));
    static_assert(kPLoads == 3, "three perm words per lane");
#pragma unroll
    for (int j = 0; j < kPLoads; ++j) {
      const int row = t.gather ? (int)pv[j] / p.k : t.arow0 + min(a_row[j], t.m - 1);
      o[j] = (uint32_t)row * (uint32_t)(K * 2) + (uint32_t)(a_col * 2);
    }
  };
  auto gaddr = [](const void* base, size_t ofs) {
    return reinterpret_cast<const char*>(base) + ofs;
  };
  auto dma_a = [&](int slot, bool nx, int st) {
    const char* ta = gaddr(p.a, (size_t)st * kBK * 2);
#pragma unroll
    for (int j = 0; j < kPLoads; ++j) {
      const int x = wid + kPW * j;
      gdma16(ta, nx ? a_off_nxt[j] : a_off_cur[j], slots[slot] + (x < kBM / 8 ? x : x - kPW / 2) * 64);
    }
  };
  auto load_b = [&](int slot, bool nx, int st) {
    const int k0 = st * kBK;
#pragma unroll
    for (int nb = 0; nb < kPNB; ++nb) {
      if constexpr (Q4) {
        const u32x2 qw = gld8(gaddr(nx ? nxt.q[nb] : cur.q[nb], (size_t)k0 / 2), q_off);
        qreg[slot][nb][0] = qw.x;
        qreg[slot][nb][1] = qw.y;
        // The 32-bit word holding this stage's scale (table entries are 16-byte aligned
        // and K / 128 is even here); multiply() takes its half.  QR: the row's one fp16
        // scale, reloaded each stage so the stage's load count stays the same.
        if constexpr (QR) sreg[slot][nb] = gld2(gaddr(nx ? nxt.sc[nb] : cur.sc[nb], 0), s_off);
        else sreg[slot][nb] = gld4(gaddr(nx ? nxt.sc[nb] : cur.sc[nb], (size_t)((k0 / 128) & ~1) * 2), s_off);
      } else {
        const char* br = gaddr(nx ? nxt.b[nb] : cur.b[nb], (size_t)k0 * 2);
        breg[slot][nb][0] = gld16(br, b_off);
        breg[slot][nb][1] = gld16(br + 64, b_off);
      }
    }
  };
  // Wait for B slot bs (issued kB - 1 iterations and one A group before): at most the
  // loads of the kB - 1 later iterations and this iteration's A loads stay outstanding.
  // The registers pass through the asm, so nothing reads them before the wait.
  auto wait_b = [&](int bs) {
    constexpr int n = (kB - 1) * (kPLoads + 2 * kPNB) + kPLoads;
    static_assert(n < 64, "vmcnt range");
    if constexpr (Q4) {
      asm volatile("s_waitcnt vmcnt(%4)"
                   : "+v"(qreg[bs][0][0]), "+v"(qreg[bs][0][1]), "+v"(qreg[bs][1][0]), "+v"(qreg[bs][1][1])
                   : "n"(n));
      asm volatile("" : "+v"(sreg[bs][0]), "+v"(sreg[bs][1]));
    } else {
      asm volatile("s_waitcnt vmcnt(%4)"
                   : "+v"(breg[bs][0][0]), "+v"(breg[bs][0][1]), "+v"(breg[bs][1][0]), "+v"(breg[bs][1][1])
                   : "n"(n));
    }
  };
  // Stage 8 c + u (A slot u, B slot u % kB) takes scale 4 c + u / 2: the high half of its
  // word for u = 2, 3, 6, 7.
  auto multiply = [&](int u) {
    const u32x4* la = slots[u];
    const int bs = u % kB;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8_t b[kPNB];
#pragma unroll
      for (int nb = 0; nb < kPNB; ++nb) {
        if constexpr (Q4) {
          const uint32_t sr = sreg[bs][nb];
          const uint32_t bits = ((u >> 1) & 1) ? (sr & 0xFFFF0000u) : (sr << 16);
          b[nb] = as_bf16x8(dequant_frag(qreg[bs][nb][ks], QR ? scale_f32<true>((uint16_t)sr) : __uint_as_float(bits)));
        } else {
          b[nb] = as_bf16x8(breg[bs][nb][ks]);
        }
      }
      const u32x4* lh = la + (ks ? a_rd1 : a_rd0);
#pragma unroll
      for (int i = 0; i < kPMB; ++i) {
        const bf16x8_t a = as_bf16x8(lh[i * 128]);
#pragma unroll
        for (int nb = 0; nb < kPNB; ++nb)
          acc[i][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[nb], acc[i][nb], 0, 0, 0);
      }
    }
  };
  // Int4: one k step's MFMAs with the next k step's dequantisation woven between them.  An
  // MFMA keeps the matrix unit busy 16 cycles, in which the wave issues independent VALU
  // work, so the dequantisation (~3 VALU instructions per MFMA) need not sit between the
  // weight load and the MFMAs.  Group i: its token block's MFMAs, one piece of the next
  // fragments (group 0: the nibble planes and scales; groups 1..8: one 32-bit word of the
  // two fragments each), and the A fragment read two blocks ahead; sched_barrier keeps the
  // groups in this order.  cur: this k step's fragments; next k step: stage nu, step nks.
  // The dequantised values are dequant_frag's, bit for bit.
  auto mma_q4 = [&](int u, int ks, const u32x4 (&cur_b)[kPNB], int nu, int nks, u32x4 (&nxt_b)[kPNB]) {
    const u32x4* lh = slots[u] + (ks ? a_rd1 : a_rd0);
    const int ns = nu % kB;
    bf16x8_t bc[kPNB];
#pragma unroll
    for (int nb = 0; nb < kPNB; ++nb) bc[nb] = as_bf16x8(cur_b[nb]);
    uint32_t lo[kPNB], hi[kPNB];
    float sc[kPNB], m8[kPNB];
    // Chunks of at most 128 rows skip the MFMAs of the last two row blocks (all padding).
    static_assert(kPMB == 10, "8 row blocks, then the two that chunks over 128 rows use");
    const bool full = cur.m > 128;
    bf16x8_t a0 = as_bf16x8(lh[0]), a1 = as_bf16x8(lh[128]);
#pragma unroll
    for (int i = 0; i < kPMB; ++i) {
      const bf16x8_t a = a0;
      a0 = a1;
      if (i + 2 < kPMB) a1 = as_bf16x8(lh[(i + 2) * 128]);
      if (i < 8 || full) {
#pragma unroll
        for (int nb = 0; nb < kPNB; ++nb)
          acc[i][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bc[nb], acc[i][nb], 0, 0, 0);
      }
      if (i == 0) {
#pragma unroll
        for (int nb = 0; nb < kPNB; ++nb) {
          const uint32_t q = qreg[ns][nb][nks];
          lo[nb] = q & 0x0F0F0F0Fu;
          hi[nb] = (q >> 4) & 0x0F0F0F0Fu;
          asm volatile("" : "+v"(lo[nb]), "+v"(hi[nb]));   // keep the byte planes: one conversion per value
          const uint32_t sr = sreg[ns][nb];
          const uint32_t bits = ((nu >> 1) & 1) ? (sr & 0xFFFF0000u) : (sr << 16);
          sc[nb] = QR ? scale_f32<true>((uint16_t)sr) : __uint_as_float(bits);
          m8[nb] = -8.0f * sc[nb];
        }
      } else if (i <= 4 * kPNB) {
        const int w = i - 1, nb = w / 4, b = w % 4;
        const float e = fmaf((float)((lo[nb] >> (8 * b)) & 0xFFu), sc[nb], m8[nb]);
        const float o = fmaf((float)((hi[nb] >> (8 * b)) & 0xFFu), sc[nb], m8[nb]);
        const bf16x2_t v = {(__bf16)e, (__bf16)o};   // (even k low, odd k high)
        const uint32_t d = __builtin_bit_cast(uint32_t, v);
        if (b == 0) nxt_b[nb].x = d;
        else if (b == 1) nxt_b[nb].y = d;
        else if (b == 2) nxt_b[nb].z = d;
        else nxt_b[nb].w = d;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  static_assert(!Q4 || 4 * kPNB + 1 <= kPMB, "every word of the next fragments has a group");
  // Each stage ends with this wave's A loads of the next stage landed (everything but the
  // last kPA - 1 stages' loads done: exact while only loads are outstanding, stricter right
  // after an epilogue's stores) and a raw barrier: every wave's part of the next A stage is
  // visible, and every wave is done reading the slot that the next stage refills.
  // (__syncthreads' release fence would wait for every outstanding load, vmcnt(0), to
  // cover the LDS writes of the direct loads.)
  constexpr int kOpsPerStage = kPLoads + 2 * kPNB;   // A, then B (int4: kPNB packed + kPNB scale loads)
  static_assert((kPA - 1) * kOpsPerStage < 64, "vmcnt range");
  auto barrier_raw = [&]() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  auto stage_end = [&]() {
    wait_vmcnt<(kPA - 1) * kOpsPerStage>();
    barrier_raw();
  };

  // Epilogue of a tile, staged through ring slot 7 (read by the tile's last stage; its
  // next fill is issued after the epilogue) in passes of BPP 16-row blocks, so that every
  // store is a whole 16-byte piece of an output row.  Row r's 16-byte chunk q sits at
  // chunk q ^ 2 ((r / 4) % 4): the four row groups of one fragment write land in distinct
  // banks.  C fragment: lane l holds rows 4 (l / 16) + e of each 16-row block, column
  // l % 16; its rows' swizzle is 2 (l / 16).
  auto epilogue = [&](const PTile& t, auto up_tag) {
    constexpr bool UP = decltype(up_tag)::value;
    constexpr int TCB = UP ? 2 * kPUpCols : 2 * kPDnCols;   // bytes per staged row
    constexpr int BPP = UP ? 5 : 2;                         // 16-row blocks per pass
    constexpr int RPP = 16 * BPP, CPR = TCB / 16;
    static_assert(RPP * TCB <= kPSlot * 16 && kPMB % BPP == 0, "a pass fits in one ring slot");
    char* stg = reinterpret_cast<char*>(slots[kPR - 1]);
    const int sw = 2 * (lane >> 4), rl = 4 * (lane >> 4);
    int cb[kPNB];
#pragma unroll
    for (int nb = 0; nb < kPNB; ++nb) {
      const int col = UP ? wid * 16 + lrow : wid * 32 + nb * 16 + lrow;
      cb[nb] = rl * TCB + ((col >> 3) ^ sw) * 16 + (col & 7) * 2;
    }
#pragma unroll
    for (int P = 0; P < kPMB / BPP; ++P) {
#pragma unroll
      for (int ii = 0; ii < BPP; ++ii) {
        const int i = P * BPP + ii;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          char* rowp = stg + (ii * 16 + e) * TCB;
          // Hardware conversions (round to nearest even), two values each.
          if constexpr (UP) {
            *reinterpret_cast<uint16_t*>(rowp + cb[0]) = swiglu_bits_hw(acc[i][0][e], acc[i][1][e]);
          } else {
            static_assert(kPNB == 2, "one conversion per row of the wave's two weight blocks");
            const uint32_t w = bf16x2_bits_hw(acc[i][0][e], acc[i][1][e]);
            *reinterpret_cast<uint16_t*>(rowp + cb[0]) = (uint16_t)w;
            *reinterpret_cast<uint16_t*>(rowp + cb[1]) = (uint16_t)(w >> 16);
          }
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      barrier_raw();
      for (int x = tid; x < RPP * CPR; x += 64 * kPW) {
        const int rr = x / CPR, qc = x - rr * CPR, row = P * RPP + rr;
        const u32x4 v = *reinterpret_cast<const u32x4*>(stg + rr * TCB + ((qc ^ (2 * ((rr >> 2) & 3))) * 16));
        if (row < t.m) *reinterpret_cast<u32x4*>(t.o + (size_t)row * p.N + qc * 8) = v;
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      barrier_raw();
    }
  };

  cur = tile(0);
  nxt = tile(min(1, ntile - 1));
  fetch_perm(pv_cur, cur);
  fetch_perm(pv_nxt, nxt);
  wait_vmcnt<0>();
  a_offsets(a_off_cur, pv_cur, cur);
  a_offsets(a_off_nxt, pv_nxt, nxt);
  // Prologue: the kPR iterations before stage 0, in the loop's own issue order (iteration
  // v - kPR requests A stage v - 1 and B stage v - kB), so the loads in flight at the top
  // of the loop stand exactly as they do after every later cycle.
#pragma unroll
  for (int v = 0; v < kPR; ++v) {
    if (v >= 1) dma_a(v - 1, false, v - 1);
    if (v >= kPR - kB) load_b(v - (kPR - kB), false, v - (kPR - kB));
  }
  stage_end();
  // Int4: stage 0's B loads landed (the kB - 1 later B stages and their A loads may still be
  // in flight) and its first k step's fragments formed; every later stage finds its first
  // fragments formed during the previous stage's second k step.
  u32x4 bq4[kPNB];
  if constexpr (Q4) {
    wait_vm_regs<(kB - 1) * kOpsPerStage>(qreg[0][0][0], qreg[0][0][1], qreg[0][1][0], qreg[0][1][1]);
    asm volatile("" : "+v"(sreg[0][0]), "+v"(sreg[0][1]));
#pragma unroll
    for (int nb = 0; nb < kPNB; ++nb) {
      const uint32_t sr = sreg[0][nb];
      bq4[nb] = dequant_frag(qreg[0][nb][0], QR ? scale_f32<true>((uint16_t)sr) : __uint_as_float(sr << 16));
    }
  }
  // Stage st of tile j (A slot st % kPR, B slot st % kB): refill the A slot read at the
  // previous stage with stage st + kPA, multiply, refill this stage's B slot with stage
  // st + kB; stages past the tile's end are the next tile's first ones (for the last
  // tile: its own first stages again, never multiplied).  K / 64 is a multiple of kPR, so
  // tiles start on a cycle boundary and every load is unconditional.
  auto cycle = [&](int st0, auto tail_tag) {
    constexpr bool kTail = decltype(tail_tag)::value;   // the tile's last cycle
#pragma unroll
    for (int u = 0; u < kPR; ++u) {
      const int sa = st0 + u + kPA, sb = st0 + u + kB;
      const bool na = kTail && u + kPA >= kPR, nb = kTail && u + kB >= kPR;   // past the tile's end
      dma_a((u + kPA) % kPR, na, na ? sa - nk : sa);
      if constexpr (Q4) {
        // k step 0 (fragments formed before) forming k step 1's; then, once stage u + 1's B
        // loads have landed (issued kB - 1 stages ago: only the kB - 2 later B stages with
        // their A loads and this stage's A loads may still be outstanding), k step 1 forming
        // stage u + 1's first.
        u32x4 q1[kPNB];
        mma_q4(u, 0, bq4, u, 1, q1);
        const int n1 = (u + 1) % kB;
        wait_vm_regs<(kB - 2) * kOpsPerStage + kPLoads>(qreg[n1][0][0], qreg[n1][0][1], qreg[n1][1][0],
                                                            qreg[n1][1][1]);
        asm volatile("" : "+v"(sreg[n1][0]), "+v"(sreg[n1][1]));
        mma_q4(u, 1, q1, u + 1, 0, bq4);
      } else {
        wait_b(u % kB);
        multiply(u);
      }
      load_b(u % kB, nb, nb ? sb - nk : sb);
      stage_end();
    }
  };
  for (int j = 0; j < ntile; ++j) {
    for (int st0 = 0; st0 < nk - kPR; st0 += kPR) cycle(st0, std::false_type{});
    // The next tile's perm entries were fetched before this tile's first stage: the
    // nk - kPR >= kPR stage waits since then leave only the last kPA - 1 stages' loads
    // outstanding.  (A gathering launch therefore needs K >= 2 kPR stages; the host sends
    // K = 512 gathers to the register-staged kernel.)
    a_offsets(a_off_nxt, pv_nxt, nxt);
    cycle(nk - kPR, std::true_type{});
    if (p.up) epilogue(cur, std::true_type{});
    else epilogue(cur, std::false_type{});
    zero_acc();
    cur = nxt;
    nxt = tile(min(j + 2, ntile - 1));
#pragma unroll
    for (int q = 0; q < kPLoads; ++q) a_off_cur[q] = a_off_nxt[q];
    fetch_perm(pv_nxt, nxt);
  }
  wait_vmcnt<0>();   // the last, unused stages landed before the block's LDS is released
}

// ---------------------------------------------------------------- grouped GEMM, whole-line weights
// Exact-bf16 twin of k_grouped_gemm_p (same tiles, descriptors, tile order and outputs), built
// around how HBM serves the weights: a load instruction reading 16 rows x 64 bytes (an MFMA
// fragment) streams at ~5-6 TB/s, one reading whole 128-byte lines of 8 rows at ~7 TB/s.
//   Weights: per 64-wide K stage a wave reads its 32 rows x 128 bytes with 4 whole-line loads
//   (load i, lane l: row 8 i + l / 8, bytes 16 (l % 8)), kWB stages ahead in registers.  At
//   its stage the wave writes them to its own 4 KB LDS region, row r's 16-byte chunk c at
//   chunk c ^ (r % 8), and reads them back as MFMA fragments (16 rows, one chunk): the
//   swizzle of the A slots, conflict-free both ways.  Only the wave itself touches its
//   region, and one wave's LDS operations complete in order.
//   A: as in k_grouped_gemm_p (direct global -> LDS loads of whole rows), in a ring of kWAS
//   slots requested kWA stages ahead; the slot is a run-time index (stage % kWAS).
// Iteration g: request A stage g + kWA; wait for weight stage g; its registers to the region;
// request weight stage g + kWB into them; 40 MFMAs; wait for A stage g + 1; barrier.
// K: a multiple of 4 stages (256) and at least 8 stages (the next tile's perm words, requested
// after a tile's epilogue, are used before its last cycle, 4 stage waits later).
// WB: weight stages in registers (the unrolled cycle; 4, or 5 where K / 64 is a multiple of
// 5), A stages requested as far ahead (every request past a tile's end falls in its last
// cycle), WB + 1 A ring slots.
constexpr int kWBLoads = 2 * kPNB;            // weight loads per wave per stage (8 rows each)
constexpr int kWReg = 16 * kPNB * 8;          // u32x4 per wave region (32 rows x 128 B)
constexpr int kWOps = kPLoads + kWBLoads;     // vector memory operations per stage

template <bool UP, int WB>
__global__ __launch_bounds__(64 * kPW, 1) void k_grouped_gemm_w(GemmParams p) {
  constexpr int kWB = WB, kWA = WB, kWAS = WB + 1;
  static_assert(kWBLoads + (kWA - 1) * kWOps < 64 && (kWB - 1) * kWOps + kPLoads < 64, "vmcnt range");
  static_assert((kWAS * kPSlot + kPW * kWReg) * 16 <= 160 * 1024, "LDS");
  __shared__ u32x4 lA[kWAS * kPSlot];
  __shared__ u32x4 lB[kPW * kWReg];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = p.K;
  u32x4* const reg = lB + wid * kWReg;

  const int c_lo = sload1(p.tile_start + p.group_lo);
  const int c_hi = sload1(p.tile_start + p.group_hi);
  const int total = (c_hi - c_lo) * p.n_ntiles;
  const int nbx = (int)gridDim.x >> 3;
  const int xcd = (int)blockIdx.x & 7, qb = (int)blockIdx.x >> 3;
  const int per_xcd = (total + 7) / 8;
  const int f0 = xcd * per_xcd + qb;
  const int f_end = min(total, (xcd + 1) * per_xcd);
  if (f0 >= f_end) return;
  const int ntile = (f_end - f0 + nbx - 1) / nbx;

  auto tile = [&](int j) {
    const int f = f0 + j * nbx;
    const int mt = c_lo + f / p.n_ntiles, nt = f % p.n_ntiles;
    const i32x4 d = sload4(p.desc + mt);
    const int g = d.x, row0 = d.z;
    const bool shared = g == p.E;
    PTile t;
    t.m = d.y;
    t.gather = p.up && !shared;
    t.arow0 = (!p.up && shared ? p.shared_row0 : 0) + row0;
    const int c0 = p.up ? nt * kPUpCols + wid * 16 : nt * kPDnCols + wid * 32;
    if (p.up) t.o = p.out + (size_t)(shared ? p.shared_row0 + row0 : row0) * p.N + nt * kPUpCols;
    else t.o = (shared ? p.out_sh : p.out) + (size_t)row0 * p.N + nt * kPDnCols;
    const uint16_t *w0, *w1;
    if (shared) {
      w0 = p.shw0;
      w1 = p.up ? p.shw1 : p.shw0;
    } else {
      w0 = w1 = reinterpret_cast<const uint16_t*>(sload_ptr(p.table + 2 * g + (p.up ? 0 : 1)));
    }
#pragma unroll
    for (int nb = 0; nb < kPNB; ++nb) {
      const int wr = p.up ? ((nb && !shared) ? p.I : 0) + c0 : c0 + 16 * nb;
      t.b[nb] = (nb ? w1 : w0) + (size_t)wr * K;
      t.q[nb] = nullptr;
      t.sc[nb] = nullptr;
    }
    return t;
  };

  PTile cur, nxt;
  // Lane constants.  A: load j covers rows 8 x .. 8 x + 7 (x = wid + 8 j, the last four
  // repeating 16..19); weights: load 2 nb + h covers rows 16 nb + 8 h + lane / 8 of the
  // wave's two blocks, bytes 16 (lane % 8).
  const int lrow = lane & 15;
  int a_row[kPLoads];
#pragma unroll
  for (int j = 0; j < kPLoads; ++j) {
    const int x = wid + kPW * j;
    a_row[j] = 8 * (x < kBM / 8 ? x : x - kPW / 2) + (lane >> 3);
  }
  const int a_col = 8 * ((lane & 7) ^ (lane >> 3));
  const int rd0 = lrow * 8 + ((lane >> 4) ^ (lrow & 7));          // fragment chunk, k 0..31
  const int rd1 = lrow * 8 + ((4 + (lane >> 4)) ^ (lrow & 7));    // k 32..63
  const int wr_off = (lane >> 3) * 8 + ((lane & 7) ^ (lane >> 3)); // region chunk of load i: + 64 i
  uint32_t b_off[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) b_off[h] = (uint32_t)(((8 * h + (lane >> 3)) * K + (lane & 7) * 8) * 2);

  f32x4 acc[kPMB][kPNB];
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < kPMB; ++i)
#pragma unroll
      for (int nb = 0; nb < kPNB; ++nb) acc[i][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  zero_acc();

  u32x4 breg[kWB][kWBLoads];
  const int nk = K / kBK;   // a multiple of kWB, at least 2 kWB
  uint32_t a_off_cur[kPLoads], a_off_nxt[kPLoads];
  uint32_t pv_cur[kPLoads], pv_nxt[kPLoads];
  // Always kPLoads loads (tiles without a gather read perm[0]): the waits count them.
  auto fetch_perm = [&](uint32_t* pv, const PTile& t) {
    const int32_t* pp = p.perm + (t.gather ? t.arow0 : 0);
#pragma unroll
    for (int j = 0; j < kPLoads; ++j) pv[j] = gld4(pp, t.gather ? (uint32_t)(min(a_row[j], t.m - 1) * 4) : 0u);
  };
  auto a_offsets = [&](uint32_t* o, uint32_t* pv, const PTile& t) {
    asm volatile("" : "+v"(pv[0]), "+v"(pv[1]), "+v"(pv[2]));
    static_assert(kPLoads == 3, "three perm words per lane");
#pragma unroll
    for (int j = 0; j < kPLoads; ++j) {
      const int row = t.gather ? (int)pv[j] / p.k : t.arow0 + min(a_row[j], t.m - 1);
      o[j] = (uint32_t)row * (uint32_t)(K * 2) + (uint32_t)(a_col * 2);
    }
  };
  auto gaddr = [](const void* base, size_t ofs) { return reinterpret_cast<const char*>(base) + ofs; };
  auto dma_a = [&](int slot, bool nx, int st) {
    const char* ta = gaddr(p.a, (size_t)st * kBK * 2);
    u32x4* const s = lA + slot * kPSlot;
#pragma unroll
    for (int j = 0; j < kPLoads; ++j) {
      const int x = wid + kPW * j;
      gdma16(ta, nx ? a_off_nxt[j] : a_off_cur[j], s + (x < kBM / 8 ? x : x - kPW / 2) * 64);
    }
  };
  auto load_b = [&](int bs, bool nx, int st) {
    const size_t k0 = (size_t)st * kBK * 2;
#pragma unroll
    for (int nb = 0; nb < kPNB; ++nb) {
      const char* br = gaddr(nx ? nxt.b[nb] : cur.b[nb], k0);
      breg[bs][2 * nb] = gld16(br, b_off[0]);
      breg[bs][2 * nb + 1] = gld16(br, b_off[1]);
    }
  };
  // Wait for weight stage bs (requested kWB - 1 iterations and one A group before, plus X
  // operations of an epilogue in between).  The registers pass through the asm, so nothing
  // reads them before the wait.
  // Stores per thread in one epilogue (up: 2 passes x 3, down: 2 passes x 5); the first 4
  // iterations of the next tile add them and the next tile's perm loads (kXH) to their waits.
  constexpr int kEpiStores = UP ? 6 : 10;
  constexpr int kXH = kEpiStores + kPLoads;
  auto wait_b = [&](int bs, bool head) {
    constexpr int n = (kWB - 1) * kWOps + kPLoads;
    static_assert(kWBLoads == 4 && n + kXH < 64, "four weight registers per stage; vmcnt range");
    if (head)
      asm volatile("s_waitcnt vmcnt(%4)"
                   : "+v"(breg[bs][0]), "+v"(breg[bs][1]), "+v"(breg[bs][2]), "+v"(breg[bs][3])
                   : "n"(n + kXH));
    else
      asm volatile("s_waitcnt vmcnt(%4)"
                   : "+v"(breg[bs][0]), "+v"(breg[bs][1]), "+v"(breg[bs][2]), "+v"(breg[bs][3])
                   : "n"(n));
  };
  const uint32_t wr_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)(reg + wr_off);
  auto to_region = [&](int bs) {
    dsw16<0 * 1024>(wr_lds, breg[bs][0]);
    dsw16<1 * 1024>(wr_lds, breg[bs][1]);
    dsw16<2 * 1024>(wr_lds, breg[bs][2]);
    dsw16<3 * 1024>(wr_lds, breg[bs][3]);
  };
  auto multiply = [&](int aslot) {
    const u32x4* la = lA + aslot * kPSlot;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int rd = ks ? rd1 : rd0;
      bf16x8_t b[kPNB];
#pragma unroll
      for (int nb = 0; nb < kPNB; ++nb) b[nb] = as_bf16x8(reg[nb * 128 + rd]);
      auto blocks = [&](int i0, int i1) {
#pragma unroll
        for (int i = i0; i < i1; ++i) {
          const bf16x8_t a = as_bf16x8(la[i * 128 + rd]);
#pragma unroll
          for (int nb = 0; nb < kPNB; ++nb)
            acc[i][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[nb], acc[i][nb], 0, 0, 0);
        }
      };
      // Down: chunks of at most 128 rows (about half the groups at ~128 tokens per expert)
      // skip the last two row blocks, all padding (down 387 -> 369 us at T=4096; the up
      // GEMM showed no gain and keeps one straight-line schedule).
      static_assert(kPMB == 10, "8 row blocks, then the two that chunks over 128 rows use");
      blocks(0, 8);
      if (UP || cur.m > 128) blocks(8, kPMB);
    }
  };
  auto barrier_raw = [&]() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // End of stage g: this wave's part of A stage g + 1 landed (requested kWA - 1 iterations
  // before, followed by that iteration's weight loads and kWA - 1 whole iterations), then a
  // raw barrier (every wave's part visible; every wave done reading the slot refilled next).
  auto stage_end = [&](bool head) {
    constexpr int n = kWBLoads + (kWA - 1) * kWOps;
    static_assert(n + kXH < 64, "vmcnt range");
    if (head) wait_vmcnt<n + kXH>();
    else wait_vmcnt<n>();
    barrier_raw();
  };

  // Epilogue in two passes of five 16-row blocks, row r's 16-byte chunk q at chunk
  // q ^ 2 ((r / 4) % 4); C fragment lane l holds rows 4 (l / 16) + e, column l % 16.
  // Staging: the wave regions (32 KB, free between a tile's last stage and the next tile's
  // first) hold the pass's first kStgRows rows, the A ring slot
  // that no load targets during the epilogue (the one the tile's last stage used; its refill
  // is requested in the next tile's first iteration) the rest.
  auto epilogue = [&](const PTile& t, int free_slot) {
    constexpr int TCB = UP ? 2 * kPUpCols : 2 * kPDnCols;
    constexpr int BPP = 5;
    constexpr int RPP = 16 * BPP, CPR = TCB / 16;
    constexpr int NST = (RPP * CPR + 64 * kPW - 1) / (64 * kPW);
    constexpr int kStgRows = kPW * kWReg * 16 / TCB;
    static_assert(kPMB % BPP == 0 && RPP <= kStgRows + kPSlot * 16 / TCB, "a pass fits in the staging");
    static_assert(NST * 64 * kPW / CPR <= kStgRows + kPSlot * 16 / TCB, "reads past the pass stay in it");
    static_assert(NST * (kPMB / BPP) == kEpiStores, "stores per thread per epilogue");
    char* const stg = reinterpret_cast<char*>(lB);
    char* const stg2 = reinterpret_cast<char*>(lA + free_slot * kPSlot);
    auto rowp = [&](int r) { return r < kStgRows ? stg + r * TCB : stg2 + (r - kStgRows) * TCB; };
    const int sw = 2 * (lane >> 4), rl = 4 * (lane >> 4);
    int cb[kPNB];
#pragma unroll
    for (int nb = 0; nb < kPNB; ++nb) {
      const int col = UP ? wid * 16 + lrow : wid * 32 + nb * 16 + lrow;
      cb[nb] = ((col >> 3) ^ sw) * 16 + (col & 7) * 2;
    }
#pragma unroll
    for (int P = 0; P < kPMB / BPP; ++P) {
#pragma unroll
      for (int ii = 0; ii < BPP; ++ii) {
        const int i = P * BPP + ii;
        if (16 * i >= t.m) continue;   // padding rows only (their stores go to the sink)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          char* const row = rowp(ii * 16 + rl + e);
          if constexpr (UP) {
            *reinterpret_cast<uint16_t*>(row + cb[0]) = swiglu_bits_hw(acc[i][0][e], acc[i][1][e]);
          } else {
            // both columns' values in one hardware conversion (round to nearest even)
            static_assert(kPNB == 2, "two column blocks per wave");
            const uint32_t pk = __builtin_bit_cast(uint32_t, bf16x2_hw{(__bf16)acc[i][0][e], (__bf16)acc[i][1][e]});
            *reinterpret_cast<uint16_t*>(row + cb[0]) = (uint16_t)pk;
            *reinterpret_cast<uint16_t*>(row + cb[1]) = (uint16_t)(pk >> 16);
          }
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      barrier_raw();
      // Exactly kEpiStores / passes stores per thread and pass, rows past the tile (and
      // places past the pass) redirected to the sink: the next tile's first waits count them.
#pragma unroll 1
      for (int q = 0; q < NST; ++q) {
        const int x = tid + q * 64 * kPW;
        const int rr = x / CPR, qc = x - rr * CPR, row = P * RPP + rr;
        const u32x4 v = *reinterpret_cast<const u32x4*>(rowp(rr) + ((qc ^ (2 * ((rr >> 2) & 3))) * 16));
        const bool ok = x < RPP * CPR && row < t.m;
        *reinterpret_cast<u32x4*>(ok ? t.o + (size_t)row * p.N + qc * 8 : p.sink) = v;
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      barrier_raw();
    }
  };

  cur = tile(0);
  nxt = tile(min(1, ntile - 1));
  fetch_perm(pv_cur, cur);
  wait_vmcnt<0>();
  a_offsets(a_off_cur, pv_cur, cur);
  // Prologue: iterations -kWA .. -1 in the loop's issue order (iteration v requests A stage
  // v + kWA, then weight stage v + kWB), then what an epilogue leaves between a tile's last
  // cycle and the next tile's first (kEpiStores stores, here to the sink, and the next
  // tile's perm loads): every tile starts with the same operations in flight.
#pragma unroll
  for (int v = -kWA; v < 0; ++v) {
    dma_a(v + kWA, false, v + kWA);
    load_b(v + kWB, false, v + kWB);
  }
  {
    const uint64_t sk = (uint64_t)(uintptr_t)p.sink;
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int q = 0; q < kEpiStores; ++q) asm volatile("global_store_dwordx4 %0, %1, off" : : "v"(sk), "v"(z) : "memory");
  }
  fetch_perm(pv_nxt, nxt);
  stage_end(true);
  // Stage counter continuous over tiles: A slot (stage % kWAS), weight slot (stage % kWB).
  // Stages past a tile's end are the next tile's first ones (the last tile: its own first
  // stages again, never multiplied); nk is a multiple of kWB, so tiles start on a cycle.
  int aslot = 0;   // A slot of this iteration's stage; its A request goes to the slot before
  // kHead: a tile's first cycle; its weight stages 0..3 and A stages 1..3 were requested
  // before the previous epilogue's stores and this tile's successor's perm loads (kXH).
  auto cycle = [&](int st0, auto tail_tag, auto head_tag) {
    constexpr bool kTail = decltype(tail_tag)::value, kHead = decltype(head_tag)::value;
    static_assert(!(kTail && kHead), "a tile has at least two cycles");
#pragma unroll
    for (int u = 0; u < kWB; ++u) {
      const int sa = st0 + u + kWA, sb = st0 + u + kWB;   // past the end exactly in the tail
      const int wslot = aslot == 0 ? kWAS - 1 : aslot - 1;
      dma_a(wslot, kTail, kTail ? sa - nk : sa);
      wait_b(u, kHead);                    // weight stage u: before the epilogue
      to_region(u);
      load_b(u, kTail, kTail ? sb - nk : sb);
      multiply(aslot);
      stage_end(kHead && u + 1 < kWB);     // A stage u + 1: before the epilogue for u + 1 < kWB
      aslot = aslot == kWAS - 1 ? 0 : aslot + 1;
    }
  };
  for (int j = 0; j < ntile; ++j) {
    cycle(0, std::false_type{}, std::true_type{});
    for (int st0 = kWB; st0 < nk - kWB; st0 += kWB) cycle(st0, std::false_type{}, std::false_type{});
    a_offsets(a_off_nxt, pv_nxt, nxt);
    cycle(nk - kWB, std::true_type{}, std::false_type{});
    epilogue(cur, aslot == 0 ? kWAS - 1 : aslot - 1);
    zero_acc();
    cur = nxt;
    nxt = tile(min(j + 2, ntile - 1));
#pragma unroll
    for (int q = 0; q < kPLoads; ++q) a_off_cur[q] = a_off_nxt[q];
    fetch_perm(pv_nxt, nxt);
  }
  wait_vmcnt<0>();
}

// ---------------------------------------------------------------- combine
// One wave per token; lane owns 8 columns per 512-column chunk.  The GEMMs leave each
// assignment's expert output and the shared expert's output unscaled (bf16 of the fp32
// accumulator); this kernel applies the routing weight and the shared gate, each product
// rounded to bf16, then accumulates in the reference's order (the token's experts
// ascending, ties in slot order, then the shared expert), rounding to bf16 after every
// addition.  Lanes 0..k-1 read the token's k entries at once and rank them.  NSPLIT waves
// share a token, wave j taking chunks j MAXC .. j MAXC + MAXC - 1 (few tokens: one chunk per
// wave).
template <int MAXC, int MAXK>
__global__ __launch_bounds__(256) void k_combine(const int32_t* ids32, const int64_t* ids64,
                                                 const int32_t* __restrict__ inv, const uint16_t* __restrict__ ch,
                                                 const float* __restrict__ wf, const uint16_t* __restrict__ wb,
                                                 const uint16_t* __restrict__ sh, const float* __restrict__ gs,
                                                 const uint16_t* __restrict__ resid, int T, int H, int E, int k,
                                                 uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int nsplit = (((H + 511) / 512) + MAXC - 1) / MAXC;
  const int wv = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int t = wv / nsplit, cbase = (wv - t * nsplit) * MAXC * 512;
  if (t >= T) return;
  int e = 0x7FFFFFFF, r = 0;
  float w = 0.f;
  bool valid = false;
  if (lane < k) {
    const size_t j = (size_t)t * k + lane;
    e = load_id(ids32, ids64, j);
    r = inv[j];
    w = wf ? wf[j] : bf16_to_f32(wb[j]);
    valid = e >= 0 && e < E && r >= 0;
    if (!valid) e = 0x7FFFFFFF;
  }
  int rank = 0;                       // position among the valid entries, by (expert, slot)
  for (int s2 = 0; s2 < k; ++s2) {
    const int e2 = __shfl(e, s2);
    rank += (e2 < e) || (e2 == e && s2 < lane);
  }
  const uint64_t vmask = __ballot(valid);
  const int n = __popcll(vmask);
  float acc[MAXC][8];
#pragma unroll
  for (int c = 0; c < MAXC; ++c)
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[c][q] = 0.f;
  // a = bf16(a + bf16(x * wt)) per column; the roundings two columns per hardware
  // conversion (round to nearest even, as the bit-operation form).
  auto add = [&](float* a, const u32x4 v, float wt) {
    const float x[8] = {bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y),
                        bf16_lo(v.z), bf16_hi(v.z), bf16_lo(v.w), bf16_hi(v.w)};
#pragma unroll
    for (int q = 0; q < 8; q += 2) {
      float p0 = x[q] * wt, p1 = x[q + 1] * wt;
      rbf16x2_hw(p0, p1);
      float s0 = a[q] + p0, s1 = a[q + 1] + p1;
      rbf16x2_hw(s0, s1);
      a[q] = s0;
      a[q + 1] = s1;
    }
  };
  // The entries in rank order (wave-uniform), then per chunk every row's load issued before
  // the additions, which stay in rank order.
  int rows[MAXK];
  float wr[MAXK];
#pragma unroll
  for (int j = 0; j < MAXK; ++j) {
    const int src = __ffsll((unsigned long long)__ballot(valid && rank == j)) - 1;
    rows[j] = j < n ? __shfl(r, src) : 0;
    wr[j] = j < n ? __shfl(w, src) : 0.f;
  }
  const float gv = sh ? gs[t] : 0.f;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int col = cbase + c * 512 + lane * 8;
    if (col >= H) continue;
    u32x4 v[MAXK];
#pragma unroll
    for (int j = 0; j < MAXK; ++j)
      if (j < n) v[j] = ld16(ch + (size_t)rows[j] * H + col);
    const u32x4 vs = sh ? ld16(sh + (size_t)t * H + col) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < MAXK; ++j)
      if (j < n) add(acc[c], v[j], wr[j]);
    if (sh) add(acc[c], vs, gv);
    if (resid) {   // the layer's residual add: bf16(h + y)
      const u32x4 hv = ld16(resid + (size_t)t * H + col);
      const float hx[8] = {bf16_lo(hv.x), bf16_hi(hv.x), bf16_lo(hv.y), bf16_hi(hv.y),
                           bf16_lo(hv.z), bf16_hi(hv.z), bf16_lo(hv.w), bf16_hi(hv.w)};
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[c][q] = hx[q] + acc[c][q];
    }
    u32x4 o;
    o.x = bf16x2_bits_hw(acc[c][0], acc[c][1]);
    o.y = bf16x2_bits_hw(acc[c][2], acc[c][3]);
    o.z = bf16x2_bits_hw(acc[c][4], acc[c][5]);
    o.w = bf16x2_bits_hw(acc[c][6], acc[c][7]);
    *reinterpret_cast<u32x4*>(out + (size_t)t * H + col) = o;
  }
}

// ---------------------------------------------------------------- driver
int dispatch_launch(const int32_t* ids32, const int64_t* ids64, int T, int k, int E, int shared_rows,
                    int32_t* offsets, int32_t* perm, int32_t* inv, int32_t* tile_start, uint32_t* err,
                    hipStream_t s, int4* desc) {
  if ((long)T * k > kScatterMaxN) return TMOE_ERR_SHAPE;
  hipLaunchKernelGGL(k_dispatch_count, dim3(1), dim3(1024), 0, s, ids32, ids64, T, k, E, shared_rows, offsets,
                     tile_start, inv, err, desc);
  hipLaunchKernelGGL(k_dispatch_scatter, dim3(E), dim3(1024), 0, s, ids32, ids64, T, k, offsets, perm, inv);
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

int prefill_launch(const uint16_t* x, int T, const int32_t* ids32, const int64_t* ids64, const float* wf,
                   const uint16_t* wb, const uint64_t* table, const uint16_t* sh_gate, const uint16_t* sh_up,
                   const uint16_t* sh_down, const float* gs, int H, int E, int I, int k, int Is, uint16_t* out,
                   void* ws, hipStream_t s, int q4, const uint16_t* resid, uint32_t* err) {
  // q4: 0 bf16 experts, 1 int4 with group-128 bf16 scales, 2 int4 with per-row fp16 scales.
  const bool has_sh = sh_gate != nullptr;
  const bool qr = q4 == 2;
  if (H % 128 || I % 64 || E > 1023 || (has_sh && Is != I)) return TMOE_ERR_SHAPE;
  if (q4 && I % 128) return TMOE_ERR_SHAPE;   // int4: every 64-wide K stage inside one 128-column group
  const Ws L = ws_layout(T, H, E, I, k, Is);
  int32_t* offsets = ws_ptr<int32_t>(ws, L.offsets);
  int32_t* perm = ws_ptr<int32_t>(ws, L.perm);
  int32_t* inv = ws_ptr<int32_t>(ws, L.inv);
  int32_t* tile_start = ws_ptr<int32_t>(ws, L.scratch);
  if (!err) err = ws_ptr<uint32_t>(ws, L.status) + kStatusError;
  uint16_t* act = ws_ptr<uint16_t>(ws, L.act);
  uint16_t* ch = ws_ptr<uint16_t>(ws, L.ch);
  uint16_t* sh = ws_ptr<uint16_t>(ws, L.sh);
  int4* desc = ws_ptr<int4>(ws, L.desc);
  if (int st = dispatch_launch(ids32, ids64, T, k, E, has_sh ? T : 0, offsets, perm, inv, tile_start, err, s,
                               desc))
    return st;

  const int n_groups = has_sh ? E + 1 : E;
  const long mbound = (long)T * k / kBM + (long)(E < T * k ? E : T * k) + (has_sh ? (T + kBM - 1) / kBM : 0) + 1;
  const long mshared = (T + kBM - 1) / kBM;

  // One GEMM over groups [lo, hi): bf16 weights, or int4 routed weights (the shared
  // group, always bf16, then gets a launch of its own).
  // The persistent kernel takes K in whole cycles of kPR stages (H and I multiples of 512),
  // covers 128 activation columns (up) or 256 output columns (down) per tile and addresses
  // A rows with 32-bit byte offsets; other shapes take the register-staged kernel (64 and
  // 128 columns).
  const int kcyc = kBK * kPR;
  const bool persistent = H % kcyc == 0 && I % kcyc == 0 && I % kPUpCols == 0 && H % kPDnCols == 0 &&
                          (size_t)T * H * 2 < ((size_t)1 << 32) && ((size_t)T * k + T) * I * 2 < ((size_t)1 << 32);
  const int up_cols = persistent ? kPUpCols : 64, dn_cols = persistent ? kPDnCols : 128;
  static int n_cu[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return TMOE_ERR_HIP;
  if (!n_cu[dev] && hipDeviceGetAttribute(&n_cu[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return TMOE_ERR_HIP;
  const unsigned pgrid = (unsigned)(n_cu[dev] >= 8 ? n_cu[dev] / 8 * 8 : 8);
  // bf16 groups of the persistent shapes run on the whole-line kernel; TMOE_PREFILL_GEMM=frag
  // selects the fragment-load kernel for them (int4 groups always use it).
  static const bool frag = [] {
    const char* e = getenv("TMOE_PREFILL_GEMM");
    return e && !strcmp(e, "frag");
  }();
  auto gemm = [&](GemmParams g, int lo, int hi, bool routed_q4, long mchunks) {
    g.group_lo = lo;
    g.group_hi = hi;
    // The fragment-load kernel reads a tile's gathered row indices one cycle (kPR stages)
    // after requesting them, so an up GEMM it would run over K < 2 kPR stages (H = 512) runs
    // on the register-staged kernel instead, with its narrower tiles.
    const bool frag_kernel = routed_q4 || frag;
    const bool staged = !persistent || (frag_kernel && g.up && g.K < 2 * kcyc);
    if (persistent && staged) g.n_ntiles = g.up ? I / 64 : H / 128;
    const long grid = (mchunks * g.n_ntiles + 7) / 8 * 8;
    if (staged) {
      if (routed_q4 && qr)
        hipLaunchKernelGGL((k_grouped_gemm<kRing, true, true>), dim3((unsigned)grid), dim3(256), 0, s, g);
      else if (routed_q4)
        hipLaunchKernelGGL((k_grouped_gemm<kRing, true>), dim3((unsigned)grid), dim3(256), 0, s, g);
      else
        hipLaunchKernelGGL((k_grouped_gemm<kRing, false>), dim3((unsigned)grid), dim3(256), 0, s, g);
    } else if (routed_q4 && qr) {
      hipLaunchKernelGGL((k_grouped_gemm_p<true, true>), dim3(pgrid), dim3(64 * kPW), 0, s, g);
    } else if (routed_q4) {
      hipLaunchKernelGGL((k_grouped_gemm_p<true>), dim3(pgrid), dim3(64 * kPW), 0, s, g);
    } else if (frag) {
      hipLaunchKernelGGL((k_grouped_gemm_p<false>), dim3(pgrid), dim3(64 * kPW), 0, s, g);
    } else if (g.up && g.K % (5 * kBK) == 0) {
      hipLaunchKernelGGL((k_grouped_gemm_w<true, 5>), dim3(pgrid), dim3(64 * kPW), 0, s, g);
    } else if (g.up) {
      hipLaunchKernelGGL((k_grouped_gemm_w<true, 4>), dim3(pgrid), dim3(64 * kPW), 0, s, g);
    } else {
      hipLaunchKernelGGL((k_grouped_gemm_w<false, 4>), dim3(pgrid), dim3(64 * kPW), 0, s, g);
    }
  };
  GemmParams up{};
  up.a = x; up.K = H; up.gather = 1; up.offsets = offsets; up.perm = perm; up.tile_start = tile_start;
  up.T = T; up.E = E; up.k = k; up.n_groups = n_groups; up.n_ntiles = I / up_cols; up.up = 1; up.N = I; up.I = I;
  up.table = table; up.shw0 = sh_gate; up.shw1 = sh_up; up.shared_row0 = T * k; up.out = act;
  up.desc = desc;
  up.sink = reinterpret_cast<uint16_t*>(tile_start + ((E + 5) & ~3));   // past tile_start's E + 2 words
  GemmParams dn = up;
  dn.a = act; dn.K = I; dn.gather = 0; dn.n_ntiles = H / dn_cols; dn.up = 0; dn.N = H;
  dn.shw0 = sh_down; dn.shw1 = nullptr; dn.out = ch; dn.out_sh = sh;
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
  const bool split = T < 512;        // few tokens: one wave per (token, 512-column chunk)
  const dim3 gc(((size_t)T * (split ? nc : 1) + 3) / 4), bc(256);
  const uint16_t* shp = has_sh ? sh : nullptr;
  auto combine = [&](auto kern) {
    hipLaunchKernelGGL(kern, gc, bc, 0, s, ids32, ids64, inv, ch, wf, wb, shp, gs, resid, T, H, E, k, out);
  };
  const int mc = split ? 1 : nc <= 2 ? 2 : nc <= 4 ? 4 : nc <= 6 ? 6 : 8;
  if (mc == 1) {
    if (k <= 8) combine(k_combine<1, 8>);
    else combine(k_combine<1, 16>);
  } else if (k <= 8) {
    if (mc == 2) combine(k_combine<2, 8>);
    else if (mc == 4) combine(k_combine<4, 8>);
    else if (mc == 6) combine(k_combine<6, 8>);
    else combine(k_combine<8, 8>);
  } else {
    if (mc == 2) combine(k_combine<2, 16>);
    else if (mc == 4) combine(k_combine<4, 16>);
    else if (mc == 6) combine(k_combine<6, 16>);
    else combine(k_combine<8, 16>);
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
                         ws_ptr<uint32_t>(workspace, L.status) + kStatusError, (hipStream_t)stream, nullptr);
}

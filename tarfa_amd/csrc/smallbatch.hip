// Small-batch experts step (2 <= T <= 16 tokens): the reference's T > 1 path
// (tarfa/engine/fused_int4.py:227-248; channel.py:44-60; transformers' eager
// Qwen3_5MoeExperts.forward, modeling_qwen3_5_moe.py:735-757) in launches whose time is the
// weight stream of the experts the batch hits, each expert read once.
//
//   k_sb_up    one wave per (slice, 8 activation columns): 8 gate and 8 up weight rows,
//              act = bf16(bf16(silu(bf16 g)) * bf16 u)                    fused_int4.py:242
//   k_sb_down  one wave per (slice, 32 output columns), d = bf16(down) unscaled; the last
//              wave to finish a 64-column tile combines it for every token: the token's
//              entries in ascending expert id (ties in slot order), each bf16(d * w) added
//              with a bf16 rounding, then the shared expert bf16(d_s * gate)
//                                        fused_int4.py:243-244, modeling_qwen3_5_moe.py:796
//   k_sb_router  (block entry) fp32 router logits, T x E/4 one-wave blocks; the last block of
//              each token selects its top-k (modeling_qwen3_5_moe.py:768-776).  At T = 2 it also
//              runs the shared expert's gate/up and gate (they need no routing), and the up
//              launch (k_sb_up_shd) then runs the shared expert's down beside the routed up tiles.
//
// Streaming.  The slice's token rows are the MFMA A operand (v_mfma_f32_16x16x32_bf16; rows
// past the slice repeat a real row and are never written), the weight rows the B operand.
// Each load instruction reads 4 weight rows x 256 contiguous bytes (whole cache lines); the
// wave moves each 16-row x 256-byte stage through a padded LDS buffer into fragment order.
// Reading fragments straight from HBM (16 rows x 64 bytes per instruction) was measured at
// 4.6 TB/s against 7.0 TB/s for whole lines.  One-wave blocks let the dispatcher balance the
// CUs at the grain of one tile (blocks of four 80 KB tiles left some CUs a third block).
//
// Cross-block hand-offs (logits to the token's last router block, expert outputs to the
// column tile's last down block) never go through an agent-scope release fence: that writes
// back the XCD's whole L2, and hundreds of them serialise (measured: ~140 us instead of ~20
// for the down kernel).  The data are written with agent-scope atomic stores, which write
// through to memory; each wave waits for its stores to complete (s_waitcnt vmcnt(0): a
// workgroup-scope release fence only waits for LDS) before the block's arrival is counted
// with an agent-scope atomic; the last
// block reads the data with agent-scope atomic loads, which miss in its own L2.
//
// Groups and slices.  Every up block derives the groups from the T*k ids in LDS: the experts
// present in ascending id (group u), each with the bitmask of its tokens (a token that lists
// an expert twice has one row; each of its slots adds the row with its own weight, as
// index_add_ adds each (token, slot) pair).  Pairs (group, token) are numbered group-major;
// pair i's expert output lives at row i of the workspace's ch region.  A group of m tokens
// is ceil(m / 8) slices of at most 8 rows (16 tokens take two passes over that expert's
// weights).  The shared expert is one more group with all T tokens (act from pair row T*k
// on, output in sh).  Block 0 of the up kernel also writes each token's combine order (the
// pair rows and the weights of its valid entries by (expert, slot)) and the slice
// descriptors the down kernel starts from.  The grids cover the most slices T*k ids can
// make; blocks past the real slices leave at once.
//
// Activations of a slice of m rows (at I * its first pair row): fragment order, element
// (row r, column c) at ((c / 8) * m + r) * 8 + c % 8, so lane (r, q) of an MFMA reads its 8
// k-values as one 16-byte word, and a wave's part of K is one contiguous run.
#include "tmoe_gemv.h"
#include "tmoe_ws.h"

namespace tmoe {

typedef __bf16 sb_bf16x8 __attribute__((ext_vector_type(8)));
typedef sb_bf16x8 bf16x8v;
__device__ __forceinline__ sb_bf16x8 sb_frag(u32x4 v) { return __builtin_bit_cast(sb_bf16x8, v); }

constexpr int kSbSlice = 8;     // rows per slice
constexpr int kSbRouterWaves = 1;   // router: waves per block, 4 logits each

// A slice as the down kernel reads it (written by block 0 of the up kernel): shared slices
// first, then the routed slices in group order.  Entry 0 is a header: arow = slice count.
struct SbSlice {
  const uint16_t* w;          // down_proj rows of the slice's expert (or the shared expert)
  uint32_t arow;              // first element of the slice's activations
  uint16_t orow;              // first output row: pair row in ch (routed) or token in sh (shared)
  uint8_t ms;                 // rows
  uint8_t shared;
};

struct SbParams {
  const uint16_t* x;          // [T, H] bf16
  const int32_t* ids32;       // [T, k] (router output) or
  const int64_t* ids64;       //         the caller's ids
  const float* wf;            // [T, k] routing weights as fp32 (bf16 values), or
  const uint16_t* wb;         //         bf16
  const uint64_t* table;      // [E][2] gate_up [2I, H], down [H, I]
  const uint16_t* sh_gate;    // shared expert [I, H], [I, H], [H, I], gate row [H]; null: none
  const uint16_t* sh_up;
  const uint16_t* sh_down;
  const uint16_t* sh_gate_w;
  const uint16_t* resid;      // layer entry: out = bf16(resid + block); else null
  int T, H, E, I, k;
  uint16_t* act;              // workspace: activations per slice (fragment order)
  uint16_t* ch;               // [T*k, H] expert outputs per pair, unscaled
  uint16_t* sh;               // [T, H] shared expert output, before its gate
  float* gs;                  // [T] shared gate bf16(sigmoid(bf16(x . w_sg)))
  int32_t* ord_row;           // [T, k] combine order: token t's j-th entry's pair row (j < ord_n[t])
  float* ord_w;               // [T, k] and its routing weight
  int32_t* ord_n;             // [T] valid entries of token t
  uint32_t* cnt;              // down: arrival counter per column tile, one per 256-byte line
  struct SbSlice* slices;     // [1 + kSbMaxEntries + 2] header (slice count), then the down kernel's slices
  uint32_t* err;
  uint16_t* out;              // [T, H]
  int sh_pre;                 // 1: the shared expert's gate/up and gate ran in the router launch, its down
                              // runs in the up launch (the down launch's slices are the routed ones)
};

struct SbGroups {
  int ids[256];          // entry t*k + s: expert id, or -1 (the sentinel E, or invalid)
  uint32_t present[32];  // experts present (E <= 1024)
  int wpre[33];          // exclusive prefix of popcounts of present[]
  uint32_t gmask[256];   // group u: its tokens
  int gexp[256];         // group u: its expert
  int gpre[257];         // group u: its first pair
  int spre[257];         // group u: its first slice
  int sgrp[256];         // slice s: its group
  int toks[16];          // this block's slice: token of row r
  int U, NS;             // groups, slices (routed)
  int gent[256];         // group u: one of its entries
  const uint16_t* ew[256];   // entry j: its expert's gate_up rows (loaded with the id)
};

__device__ __forceinline__ int sb_load_id(const SbParams& p, int j) {
  return p.ids32 ? p.ids32[j] : (int)p.ids64[j];
}

// This wave's stores have completed (vmcnt(0)).  The hand-off stores are device-scope
// (write-through), so once complete they are visible to device-scope loads; a workgroup-scope
// release fence would not do: it compiles to an LDS wait only.
__device__ __forceinline__ void sb_stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ int sb_group_of(const SbGroups& g, int e) {
  return g.wpre[e >> 5] + __popc(g.present[e >> 5] & ((1u << (e & 31)) - 1u));
}

// Groups and slices from the ids (T*k <= 256; any block of at least 64 threads).
__device__ void sb_groups(const SbParams& p, SbGroups& g, bool duty) {
  const int tid = threadIdx.x, nthr = blockDim.x, n = p.T * p.k;
  for (int j = tid; j < 32; j += nthr) g.present[j] = 0u;
  for (int j = tid; j < 256; j += nthr) g.gmask[j] = 0u;
  int ev[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int j = tid + i * nthr;
    ev[i] = j < n ? sb_load_id(p, j) : p.E;
  }
  bool bad = false;
  const uint16_t* ew[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int j = tid + i * nthr;
    int e = ev[i];
    if (e < 0 || e >= p.E) {
      bad |= e != p.E;
      e = -1;
    }
    if (j < 256) g.ids[j] = e;
    // The expert's gate_up rows, requested now: the round trip overlaps the group work below.
    ew[i] = e >= 0 ? reinterpret_cast<const uint16_t*>(p.table[2 * e]) : nullptr;
  }
  if (bad && duty) atomicOr(p.err, (uint32_t)kErrExpertId);
  __syncthreads();
  for (int j = tid; j < n; j += nthr) {
    const int e = g.ids[j];
    if (e >= 0) atomicOr(&g.present[e >> 5], 1u << (e & 31));
  }
  __syncthreads();
  if (tid < 64) {
    int v = tid < 32 ? __popc(g.present[tid]) : 0;
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(v, d);
      if (tid >= d) v += o;
    }
    if (tid < 32) g.wpre[tid + 1] = v;
    if (tid == 0) g.wpre[0] = 0;
  }
  __syncthreads();
  for (int j = tid; j < n; j += nthr) {
    const int e = g.ids[j];
    if (e >= 0) {
      const int u = sb_group_of(g, e);
      atomicOr(&g.gmask[u], 1u << (j / p.k));
      g.gexp[u] = e;
      g.gent[u] = j;
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int j = tid + i * nthr;
    if (j < 256) g.ew[j] = ew[i];
  }
  __syncthreads();
  if (tid < 64) {
    // Four groups per lane: pair and slice counts, exclusive prefixes over the wave.
    const int U = g.wpre[32];
    int c[4], ns[4], sc = 0, ss = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int u = tid * 4 + i;
      c[i] = u < U ? __popc(g.gmask[u]) : 0;
      ns[i] = (c[i] + kSbSlice - 1) / kSbSlice;
      sc += c[i];
      ss += ns[i];
    }
    int v = sc, w = ss;
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(v, d), o2 = __shfl_up(w, d);
      if (tid >= d) {
        v += o;
        w += o2;
      }
    }
    int run = v - sc, srun = w - ss;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int u = tid * 4 + i;
      g.gpre[u] = run;
      g.spre[u] = srun;
      for (int j = 0; j < ns[i]; ++j) g.sgrp[srun + j] = u;
      run += c[i];
      srun += ns[i];
    }
    if (tid == 63) {
      g.gpre[256] = v;
      g.spre[256] = w;
      g.U = U;
      g.NS = w;
    }
  }
  __syncthreads();
}

// Tokens of this block's slice (the ranks [r0, r0 + ms) of mask) into g.toks.
__device__ __forceinline__ void sb_tokens(SbGroups& g, uint32_t mask, int r0, int ms) {
  const int tid = threadIdx.x;
  if (tid < 16 && ((mask >> tid) & 1u)) {
    const int r = __popc(mask & ((1u << tid) - 1u)) - r0;
    if (r >= 0 && r < ms) g.toks[r] = tid;
  }
  __syncthreads();
}

// Each token's valid entries ranked by (expert, slot): pair row and weight (block 0).
// The down kernel's slice descriptors (block 0 of the up kernel).
__device__ void sb_slices(const SbParams& p, const SbGroups& g) {
  const int T = p.T, I = p.I;
  const int nshs = p.sh_gate && !p.sh_pre ? (T + kSbSlice - 1) / kSbSlice : 0;
  const int total = nshs + g.NS;
  for (int si = threadIdx.x; si < total; si += blockDim.x) {
    SbSlice d;
    if (si < nshs) {
      d.w = p.sh_down;
      d.ms = (uint8_t)min(kSbSlice, T - kSbSlice * si);
      d.orow = (uint16_t)(kSbSlice * si);
      d.arow = (uint32_t)((T * p.k + kSbSlice * si) * I);
      d.shared = 1;
    } else {
      const int s = si - nshs, u = g.sgrp[s], sj = s - g.spre[u];
      d.w = reinterpret_cast<const uint16_t*>(p.table[2 * g.gexp[u] + 1]);
      d.ms = (uint8_t)min(kSbSlice, __popc(g.gmask[u]) - kSbSlice * sj);
      d.orow = (uint16_t)(g.gpre[u] + kSbSlice * sj);
      d.arow = (uint32_t)d.orow * (uint32_t)I;
      d.shared = 0;
    }
    p.slices[1 + si] = d;
  }
  if (threadIdx.x == 0) {
    SbSlice h{};
    h.arow = (uint32_t)total;
    p.slices[0] = h;
  }
}

__device__ void sb_order(const SbParams& p, const SbGroups& g) {
  const int k = p.k;
  for (int j = threadIdx.x; j < p.T * k; j += blockDim.x) {
    const int t = j / k, s = j - t * k, e = g.ids[j];
    int rank = 0, nv = 0;
    for (int s2 = 0; s2 < k; ++s2) {
      const int e2 = g.ids[t * k + s2];
      nv += e2 >= 0;
      rank += e2 >= 0 && (e2 < e || (e2 == e && s2 < s));
    }
    if (e >= 0) {
      const int u = sb_group_of(g, e);
      p.ord_row[t * k + rank] = g.gpre[u] + __popc(g.gmask[u] & ((1u << t) - 1u));
      p.ord_w[t * k + rank] = p.wf ? p.wf[j] : bf16_to_f32(p.wb[j]);
    }
    if (s == 0) p.ord_n[t] = nv;
  }
}

__device__ __forceinline__ u32x4 sb_ld_coherent(const uint16_t* p) {
  const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
  const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return u32x4{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
}

// The combine order and the shared gate as the down kernel keeps them in LDS (loaded when a
// wave starts, so the last wave of a tile combines with one round trip: its expert outputs).
struct SbOrder {
  int row[kSbMaxEntries];
  float w[kSbMaxEntries];
  int n[kSbMaxTokens];
  float gs[kSbMaxTokens];
};

// The order held in registers from the wave's start: lane l keeps entries l + 64 i.
struct SbOrderRegs {
  int row[kSbMaxEntries / 64];
  float w[kSbMaxEntries / 64];
  int n;
  float gs;
  __device__ __forceinline__ void load(const SbParams& p, int lane) {
    const int ne = p.T * p.k;
#pragma unroll
    for (int i = 0; i < kSbMaxEntries / 64; ++i) {
      const int j = lane + 64 * i;
      row[i] = j < ne ? p.ord_row[j] : 0;
      w[i] = j < ne ? p.ord_w[j] : 0.f;
    }
    n = lane < p.T ? p.ord_n[lane] : 0;
    gs = lane < p.T && p.sh_gate ? p.gs[lane] : 0.f;
  }
  __device__ __forceinline__ void store(SbOrder& o, int lane) const {
#pragma unroll
    for (int i = 0; i < kSbMaxEntries / 64; ++i) {
      o.row[lane + 64 * i] = row[i];
      o.w[lane + 64 * i] = w[i];
    }
    if (lane < kSbMaxTokens) {
      o.n[lane] = n;
      o.gs[lane] = gs;
    }
  }
};

// W 32-bit words (2 W bf16 columns) of a row: agent-scope loads (the other waves' outputs) or
// plain ones (the residual), and the store.
template <int W>
struct SbWords {
  uint32_t v[W];
};
template <int W>
__device__ __forceinline__ SbWords<W> sb_ld_words_coherent(const uint16_t* p) {
  SbWords<W> r;
  if constexpr (W == 4) {
    const u32x4 q = sb_ld_coherent(p);
    r.v[0] = q.x; r.v[1] = q.y; r.v[2] = q.z; r.v[3] = q.w;
  } else if constexpr (W == 2) {
    const uint64_t q = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    r.v[0] = (uint32_t)q; r.v[1] = (uint32_t)(q >> 32);
  } else {
    static_assert(W == 1, "1, 2 or 4 words");
    r.v[0] = __hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return r;
}
template <int W>
__device__ __forceinline__ SbWords<W> sb_ld_words(const uint16_t* p) {
  SbWords<W> r;
  if constexpr (W == 4) {
    const u32x4 q = ld16(p);
    r.v[0] = q.x; r.v[1] = q.y; r.v[2] = q.z; r.v[3] = q.w;
  } else if constexpr (W == 2) {
    const uint64_t q = *reinterpret_cast<const uint64_t*>(p);
    r.v[0] = (uint32_t)q; r.v[1] = (uint32_t)(q >> 32);
  } else {
    r.v[0] = *reinterpret_cast<const uint32_t*>(p);
  }
  return r;
}

// Combine of output columns [c0, c0 + ncols) for every token, one lane per (token, 2 W
// columns): the shared expert's output, the residual and up to 8 expert outputs (agent-scope
// loads) requested together, then added in rank order.  acc = bf16(acc + bf16(x * w)) per
// column, the roundings two columns per hardware conversion (round to nearest even, as the
// bit-operation form, which made the combine VALU-bound: ~4.5 us for the last wave of a tile at
// T=2 in a per-wave timeline, 2.4 us with the conversions and 8 columns per lane).
template <int W>
__device__ void sb_combine_w(const SbParams& p, const SbOrder& o, int c0, int ncols) {
  const int H = p.H, k = p.k, chunks = ncols / (2 * W);
  for (int job = threadIdx.x; job < p.T * chunks; job += blockDim.x) {
    const int t = job / chunks, col = c0 + (job - t * chunks) * 2 * W;
    const int nv = o.n[t];
    SbWords<W> vs{}, hv{};
    if (p.sh_gate) vs = sb_ld_words_coherent<W>(p.sh + (size_t)t * H + col);
    if (p.resid) hv = sb_ld_words<W>(p.resid + (size_t)t * H + col);
    float acc[2 * W];
#pragma unroll
    for (int i = 0; i < 2 * W; ++i) acc[i] = 0.f;
    auto add = [&](const SbWords<W>& d, float wgt) {
#pragma unroll
      for (int i = 0; i < W; ++i) {
        float p0 = bf16_lo(d.v[i]) * wgt, p1 = bf16_hi(d.v[i]) * wgt;
        rbf16x2_hw(p0, p1);
        float s0 = acc[2 * i] + p0, s1 = acc[2 * i + 1] + p1;
        rbf16x2_hw(s0, s1);
        acc[2 * i] = s0;
        acc[2 * i + 1] = s1;
      }
    };
    // Eight entries' loads in flight at a time, added in rank order.
    for (int j0 = 0; j0 < nv; j0 += 8) {
      SbWords<W> v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j0 + j < nv) v[j] = sb_ld_words_coherent<W>(p.ch + (size_t)o.row[t * k + j0 + j] * H + col);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j0 + j < nv) add(v[j], o.w[t * k + j0 + j]);
    }
    if (p.sh_gate) add(vs, o.gs[t]);
    SbWords<W> out;
#pragma unroll
    for (int i = 0; i < W; ++i) {
      float a = acc[2 * i], b = acc[2 * i + 1];
      if (p.resid) {   // the layer's residual add: bf16(h + y)
        a = bf16_lo(hv.v[i]) + a;
        b = bf16_hi(hv.v[i]) + b;
      }
      out.v[i] = bf16x2_bits_hw(a, b);
    }
    uint16_t* dst = p.out + (size_t)t * H + col;
    if constexpr (W == 4) *reinterpret_cast<u32x4*>(dst) = u32x4{out.v[0], out.v[1], out.v[2], out.v[3]};
    else if constexpr (W == 2) *reinterpret_cast<uint64_t*>(dst) = (uint64_t)out.v[0] | ((uint64_t)out.v[1] << 32);
    else *reinterpret_cast<uint32_t*>(dst) = out.v[0];
  }
}
// The fewest columns per lane that still cover the tile in one pass of the wave (each pass is a
// round trip of loads): T = 2 two columns per lane (1.4 us less per call than eight), T = 3, 4
// four, else eight (two columns at T = 4 took two passes: +0.4 us).
__device__ void sb_combine(const SbParams& p, const SbOrder& o, int c0, int ncols) {
  if (p.T * (ncols / 2) <= 64) sb_combine_w<1>(p, o, c0, ncols);
  else if (p.T * (ncols / 4) <= 64) sb_combine_w<2>(p, o, c0, ncols);
  else sb_combine_w<4>(p, o, c0, ncols);
}

// Up work of one (slice, NC activation columns) tile: NC gate and NC up weight rows over K = H
// (H / 128 stages, R in flight), act = bf16(bf16(silu(bf16 g)) * bf16 u) for the slice's ms
// token rows into the activations at arow0.  The lane's A rows: tok[j] = the token of slice
// row min(4 j + lane / 16, ms - 1).  bt, at: the wave's LDS.  NC = 8 fills the MFMA's 16
// columns; NC = 4 (rows 8-15 of B repeat rows 0-7) halves a tile's bytes, for tiles that must
// finish in fewer ring lengths.
template <int R, int NC = 8>
__device__ __forceinline__ void sb_up_tile(const SbParams& p, const uint16_t* gate, const uint16_t* up, int tile,
                                           size_t arow0, int ms, const int (&tok)[2], u32x4* bt, u32x4* at) {
  static_assert(NC == 8 || NC == 4, "8 or 4 activation columns per tile");
  constexpr int NB = NC / 2;                          // weight loads per stage (4 rows each)
  const int lane = threadIdx.x;
  const int H = p.H, nkb = H / 128;
  const int n = lane & 15, q = lane >> 4;
  const int rr = min(n, ms - 1);
  // B: load jj of a stage reads weight row 4 jj + q (gate rows 0 .. NC-1, up rows NC .. 2NC-1
  // of activation columns NC tile ..); lane (c, q) takes 16-byte chunk c of the stage's 256
  // bytes of that row: two whole cache lines per row per load.
  const uint16_t* pb[NB];
#pragma unroll
  for (int jj = 0; jj < NB; ++jj) {
    const int rw = 4 * jj + q;
    pb[jj] = (rw < NC ? gate : up) + (size_t)(tile * NC + rw % NC) * H + n * 8;
  }
  // A: load j reads chunk n of token row min(4 j + q, ms - 1) of the slice.
  const uint16_t* pa[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) pa[j] = p.x + (size_t)tok[j] * H + n * 8;
  u32x4 bq[R][NB], aq[R][2];
  auto load = [&](int slot, int st) {
#pragma unroll
    for (int jj = 0; jj < NB; ++jj) bq[slot][jj] = ld_stream(pb[jj] + st * 128);
#pragma unroll
    for (int j = 0; j < 2; ++j) aq[slot][j] = ld16(pa[j] + st * 128);
  };
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // Through LDS into MFMA fragments: lane (r, q) of MFMA i takes columns 128 s + 32 i + 8 q
  // of weight row r (B) and of token row rr (A).
  auto mult = [&](int slot) {
#pragma unroll
    for (int jj = 0; jj < NB; ++jj) bt[(4 * jj + q) * 17 + n] = bq[slot][jj];
#pragma unroll
    for (int j = 0; j < 2; ++j) at[(4 * j + q) * 17 + n] = aq[slot][j];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sb_frag(at[rr * 17 + 4 * i + q]),
                                                    sb_frag(bt[(n % (2 * NC)) * 17 + 4 * i + q]), acc, 0, 0, 0);
    // One stage's fragments live at a time (the scheduler would otherwise hoist the next
    // stage's LDS reads and cost a wave slot per SIMD).
    __builtin_amdgcn_sched_barrier(0);
  };
#pragma unroll
  for (int st = 0; st < R; ++st) load(st, st);
  for (int kb0 = 0; kb0 + R < nkb; kb0 += R) {
#pragma unroll
    for (int st = 0; st < R; ++st) {
      mult(st);
      load(st, kb0 + st + R);
    }
  }
#pragma unroll
  for (int st = 0; st < R; ++st) mult(st);
  // C: lane (n, q) holds column n (0 .. NC-1 gate, NC .. 2NC-1 up of activation column
  // NC tile + n % NC) of rows 4q .. 4q + 3; activation column c of row r lives at element
  // ((c / 8) ms + r) 8 + c % 8.
  float upv[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) upv[v] = __shfl(acc[v], lane + NC);
  if (n < NC) {
    const int c = tile * NC + n;
    uint16_t* dst = p.act + arow0 + (size_t)(c >> 3) * ms * 8 + (c & 7);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = 4 * q + v;
      if (r < ms) dst[r * 8] = f32_to_bf16(swiglu_bf16(rbf16(acc[v]), rbf16(upv[v])));
    }
  }
}

// The shared expert's gate of token t: bf16(sigmoid(bf16(x_t . w_sg))), one wave.
__device__ __forceinline__ void sb_shared_gate(const SbParams& p, int t) {
  const int lane = threadIdx.x & 63, H = p.H;
  float a = 0.f;
  for (int c = lane; c < H / 8; c += 64) a = dot8bb(ld16(p.sh_gate_w + c * 8), ld16(p.x + (size_t)t * H + c * 8), a);
  a = wave_sum(a);
  if (lane == 0) p.gs[t] = rbf16(sigmoid_f32(rbf16(a)));
}

// Shared slice sj's up tile `tile` of NC columns (rows: tokens 8 sj ..), the shared gate of
// token `gate_t` when gate_t < T.
template <int R, int NC>
__device__ __forceinline__ void sb_shared_up(const SbParams& p, int sj, int tile, int gate_t, u32x4* bt, u32x4* at) {
  const int T = p.T, I = p.I;
  const int ms = min(kSbSlice, T - kSbSlice * sj), q = (int)threadIdx.x >> 4;
  const int tok[2] = {kSbSlice * sj + min(q, ms - 1), kSbSlice * sj + min(4 + q, ms - 1)};
  sb_up_tile<R, NC>(p, p.sh_gate, p.sh_up, tile, (size_t)(T * p.k + kSbSlice * sj) * I, ms, tok, bt, at);
  if (gate_t < T) sb_shared_gate(p, gate_t);
}

// Down work of one (slice, 32 output columns) tile: two 16-column MFMA tiles sharing the A
// fragments, I / 128 stages (R in flight); d = bf16(acc) to the slice's output rows with
// 8-byte agent-scope atomic stores.  bt, at, dt: the wave's LDS.
template <int R>
__device__ __forceinline__ void sb_down_tile(const SbParams& p, const SbSlice& d, int tile, u32x4* bt, u32x4* at,
                                             uint16_t (*dt)[32]) {
  const int lane = threadIdx.x & 63;
  const int H = p.H, I = p.I, nkb = I / 128;
  const int ms = d.ms;
  const int n = lane & 15, q = lane >> 4;
  const int rr = min(n, ms - 1);
  const uint16_t* pb = d.w + (size_t)(tile * 32 + q) * I + n * 8;   // load jj: row 4 jj + q
  const uint16_t* pa[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) pa[j] = p.act + d.arow + (size_t)min(64 * j + lane, 16 * ms - 1) * 8;
  const int a_st = 128 * ms;
  u32x4 bq[R][8], aq[R][2];
  auto load = [&](int slot, int st) {
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) bq[slot][jj] = ld_stream(pb + (size_t)4 * jj * I + st * 128);
#pragma unroll
    for (int j = 0; j < 2; ++j) aq[slot][j] = ld16(pa[j] + (size_t)st * a_st);
  };
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  auto mult = [&](int slot) {
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) bt[(4 * jj + q) * 17 + n] = bq[slot][jj];
#pragma unroll
    for (int j = 0; j < 2; ++j) at[min(64 * j + lane, 16 * ms - 1)] = aq[slot][j];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bf16x8v a = sb_frag(at[(4 * i + q) * ms + rr]);
      acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, sb_frag(bt[n * 17 + 4 * i + q]), acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, sb_frag(bt[(16 + n) * 17 + 4 * i + q]), acc1, 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
#pragma unroll
  for (int st = 0; st < R; ++st) load(st, st);
  for (int kb0 = 0; kb0 + R < nkb; kb0 += R) {
#pragma unroll
    for (int st = 0; st < R; ++st) {
      mult(st);
      load(st, kb0 + st + R);
    }
  }
#pragma unroll
  for (int st = 0; st < R; ++st) mult(st);
  // C: lane (n, q) holds column n of rows 4q .. 4q + 3 of each tile.  Through LDS to 4
  // columns of one row per lane, 8-byte agent-scope atomic stores.
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    dt[4 * q + v][n] = f32_to_bf16(acc0[v]);
    dt[4 * q + v][16 + n] = f32_to_bf16(acc1[v]);
  }
  uint16_t* obase = d.shared ? p.sh : p.ch;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = lane >> 3, c = 4 * (lane & 7);           // 8 lanes per row, 32 columns
    const int rw = r + 8 * h;
    if (rw < ms) {
      const uint64_t word = *reinterpret_cast<const uint64_t*>(&dt[rw][c]);
      __hip_atomic_store(reinterpret_cast<uint64_t*>(obase + (size_t)(d.orow + rw) * H + tile * 32 + c), word,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// The shared slice sj as a down slice.
__device__ __forceinline__ SbSlice sb_shared_slice(const SbParams& p, int sj) {
  SbSlice d;
  d.w = p.sh_down;
  d.ms = (uint8_t)min(kSbSlice, p.T - kSbSlice * sj);
  d.orow = (uint16_t)(kSbSlice * sj);
  d.arow = (uint32_t)((p.T * p.k + kSbSlice * sj) * p.I);
  d.shared = 1;
  return d;
}

// Up: one wave per (slice, 8 activation columns) = 8 gate and 8 up weight rows over K = H
// (128 nkb columns, R stages in flight); block 0 also writes the combine order and the down
// kernel's slice descriptors; blocks 0 .. T-1 (shared slice 0) compute the shared gate.
template <int R>
__global__ __launch_bounds__(64) void k_sb_up(SbParams p) {
  __shared__ SbGroups g;
  __shared__ u32x4 bt[16 * 17];                       // a stage's 16 weight rows x 16 chunks, rows padded
  __shared__ u32x4 at[8 * 17];                        // a stage's token rows x 16 chunks, rows padded
  sb_groups(p, g, blockIdx.x == 0);
  if (blockIdx.x == 0) {
    sb_order(p, g);
    sb_slices(p, g);
  }
  const int lane = threadIdx.x;
  const int T = p.T, H = p.H, I = p.I;
  const int tiles = I / 8;
  const int nshs = p.sh_gate ? (T + kSbSlice - 1) / kSbSlice : 0;
  const int nkb = H / 128;
  int b = blockIdx.x, tile, sj, ms;
  uint32_t mask;
  size_t arow0;
  const uint16_t *gate, *up;
  const bool shared = b < nshs * tiles;
  if (shared) {
    sj = b / tiles;
    tile = b - sj * tiles;
    mask = (1u << T) - 1u;
    ms = min(kSbSlice, T - kSbSlice * sj);
    arow0 = (size_t)(T * p.k + kSbSlice * sj) * I;
    gate = p.sh_gate;
    up = p.sh_up;
  } else {
    b -= nshs * tiles;
    const int s = b / tiles;
    tile = b - s * tiles;
    if (s >= g.NS) return;
    const int u = g.sgrp[s];
    sj = s - g.spre[u];
    mask = g.gmask[u];
    ms = min(kSbSlice, __popc(mask) - kSbSlice * sj);
    arow0 = (size_t)(g.gpre[u] + kSbSlice * sj) * I;
    gate = g.ew[g.gent[u]];
    up = gate + (size_t)I * H;
  }
  sb_tokens(g, mask, kSbSlice * sj, ms);
  const int n = lane & 15, q = lane >> 4;
  const int rr = min(n, ms - 1);
  // B: load jj of a stage reads weight row 4 jj + q (gate rows 0-7, up rows 8-15 of
  // activation columns 8 tile ..); lane (c, q) takes 16-byte chunk c of the stage's 256
  // bytes of that row: two whole cache lines per row per load.
  const uint16_t* pb[4];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int rw = 4 * jj + q;
    pb[jj] = (rw < 8 ? gate : up) + (size_t)(tile * 8 + (rw & 7)) * H + n * 8;
  }
  // A: load j reads chunk n of token row min(4 j + q, ms - 1) of the slice.
  const uint16_t* pa[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) pa[j] = p.x + (size_t)g.toks[min(4 * j + q, ms - 1)] * H + n * 8;
  u32x4 bq[R][4], aq[R][2];
  auto load = [&](int slot, int st) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) bq[slot][jj] = ld_stream(pb[jj] + st * 128);
#pragma unroll
    for (int j = 0; j < 2; ++j) aq[slot][j] = ld16(pa[j] + st * 128);
  };
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // Through LDS into MFMA fragments: lane (r, q) of MFMA i takes columns 128 s + 32 i + 8 q
  // of weight row r (B) and of token row rr (A).
  auto mult = [&](int slot) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) bt[(4 * jj + q) * 17 + n] = bq[slot][jj];
#pragma unroll
    for (int j = 0; j < 2; ++j) at[(4 * j + q) * 17 + n] = aq[slot][j];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sb_frag(at[rr * 17 + 4 * i + q]), sb_frag(bt[n * 17 + 4 * i + q]),
                                                    acc, 0, 0, 0);
    // One stage's fragments live at a time (the scheduler would otherwise hoist the next
    // stage's LDS reads and cost a wave slot per SIMD).
    __builtin_amdgcn_sched_barrier(0);
  };
#pragma unroll
  for (int st = 0; st < R; ++st) load(st, st);
  for (int kb0 = 0; kb0 + R < nkb; kb0 += R) {
#pragma unroll
    for (int st = 0; st < R; ++st) {
      mult(st);
      load(st, kb0 + st + R);
    }
  }
#pragma unroll
  for (int st = 0; st < R; ++st) mult(st);
  // C: lane (n, q) holds column n (0-7 gate, 8-15 up of activation column 8 tile + n % 8) of
  // rows 4q .. 4q + 3.
  float upv[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) upv[v] = __shfl(acc[v], lane + 8);
  if (n < 8) {
    uint16_t* dst = p.act + arow0 + (size_t)tile * ms * 8 + n;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = 4 * q + v;
      if (r < ms) dst[r * 8] = f32_to_bf16(swiglu_bf16(rbf16(acc[v]), rbf16(upv[v])));
    }
  }
  if (shared && blockIdx.x < (unsigned)T) {            // the shared expert's gate of token blockIdx.x
    const int t = blockIdx.x;
    float a = 0.f;
    for (int c = lane; c < H / 8; c += 64) a = dot8bb(ld16(p.sh_gate_w + c * 8), ld16(p.x + (size_t)t * H + c * 8), a);
    a = wave_sum(a);
    if (lane == 0) p.gs[t] = rbf16(sigmoid_f32(rbf16(a)));
  }
}

// Up launch with sh_pre: the first blocks are the shared expert's down tiles (its activations
// came from the router launch), one per (shared slice, 32 output columns); then one wave per
// routed (slice, 8 activation columns) as in k_sb_up, block `duty` (the first routed one)
// writing the combine order and the down kernel's slice descriptors.  Three waves per SIMD
// (168 registers) keep a T=2 grid resident.
template <int R>
__global__ __launch_bounds__(64, 3) void k_sb_up_shd(SbParams p) {
  // The shared down tiles need no groups: the two uses share the block's LDS.
  struct UpLds {
    SbGroups g;
    u32x4 bt[16 * 17];                                // a stage's 16 weight rows x 16 chunks, rows padded
    u32x4 at[8 * 17];                                 // a stage's token rows x 16 chunks, rows padded
  };
  struct DnLds {
    u32x4 bt[32 * 17];
    u32x4 at[8 * 17];
    __align__(16) uint16_t dt[16][32];
  };
  __shared__ union {
    UpLds up;
    DnLds dn;
  } sm;
  const int T = p.T, H = p.H, I = p.I;
  const int tiles = I / 8;
  const int nshs = p.sh_gate ? (T + kSbSlice - 1) / kSbSlice : 0;
  const int nshd = nshs * (H / 32);
  int b = blockIdx.x;
  if (b < nshd) {
    const int sj = b / (H / 32);
    sb_down_tile<2>(p, sb_shared_slice(p, sj), b - sj * (H / 32), sm.dn.bt, sm.dn.at, sm.dn.dt);
    return;
  }
  SbGroups& g = sm.up.g;
  const bool duty = b == nshd;
  b -= nshd;
  sb_groups(p, g, duty);
  if (duty) {
    sb_order(p, g);
    sb_slices(p, g);
  }
  const int s = b / tiles, tile = b - s * tiles;
  if (s >= g.NS) return;
  const int u = g.sgrp[s];
  const int sj = s - g.spre[u];
  const uint32_t mask = g.gmask[u];
  const int ms = min(kSbSlice, __popc(mask) - kSbSlice * sj);
  const uint16_t* gate = g.ew[g.gent[u]];
  sb_tokens(g, mask, kSbSlice * sj, ms);
  const int q = (int)threadIdx.x >> 4;
  const int tok[2] = {g.toks[min(q, ms - 1)], g.toks[min(4 + q, ms - 1)]};
  sb_up_tile<R>(p, gate, gate + (size_t)I * H, tile, (size_t)(g.gpre[u] + kSbSlice * sj) * I, ms, tok, sm.up.bt,
                sm.up.at);
}

// Down: one wave per (slice, 32 output columns); the slice comes from the up kernel's
// descriptors, so a wave's first weight load issues after one descriptor read.  The last wave
// of a 64-column tile combines it.
template <int R>
__global__ __launch_bounds__(64) void k_sb_down(SbParams p) {
  __shared__ u32x4 bt[32 * 17];                       // a stage's 32 weight rows x 16 chunks, rows padded
  __shared__ u32x4 at[8 * 17];                        // a stage's activations, chunks x rows
  __shared__ __align__(16) uint16_t dt[16][32];      // the outputs, rows x columns
  __shared__ SbOrder so;                              // the combine order (for the tile's last wave)
  const int lane = threadIdx.x;
  const int H = p.H;
  const int tiles = H / 32;
  const int si = blockIdx.x / tiles, tile = blockIdx.x - si * tiles;
  const int total = (int)p.slices[0].arow;
  SbOrderRegs ordr;
  if (si >= total) {
    // No slice at all: the output is the shared expert's (or zero), plus the residual.
    if (total == 0 && si == 0 && (tile & 1) == 0) {
      ordr.load(p, lane);
      ordr.store(so, lane);
      sb_combine(p, so, tile * 32, 64);
    }
    return;
  }
  const SbSlice d = p.slices[1 + si];
  ordr.load(p, lane);
  sb_down_tile<R>(p, d, tile, bt, at, dt);
  // Arrival on the 64-column combine tile once the stores have completed; the last of its
  // 2 x (slices) waves combines it and re-zeroes the counter.
  sb_stores_done();
  const int ct = tile >> 1;
  const uint32_t arrivals = 2u * (uint32_t)total;
  uint32_t prev = 0;
  if (lane == 0) prev = __hip_atomic_fetch_add(p.cnt + ct * kLine, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = __shfl(prev, 0);
  if (prev != arrivals - 1u) return;
  ordr.store(so, lane);
  sb_combine(p, so, ct * 64, 64);
  if (lane == 0) __hip_atomic_store(p.cnt + ct * kLine, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Router logits and per-token top-k.  Block (t, y < nb) computes logits 4 y .. 4 y + 3 of token
// t and stores them with agent-scope atomic stores; the token's last block selects.  One-wave
// blocks spread the router weight's read over E / 4 CUs per token (4-wave blocks, a quarter as
// many CUs: T=2 63.4 against 62.7 us per layer).  Blocks (t, y >= nb), when sp.sh_pre, run the
// shared expert's up tiles and gate, which need no routing: (y - nb) T + t indexes the shared
// slices' tiles of 4 activation columns (R stages in flight, so a tile is two ring lengths and
// ends within the routing's latency), and tile indexes below T compute token j's gate.
template <int MAXC, int MAXEPL, int R>
__global__ __launch_bounds__(64 * kSbRouterWaves) void k_sb_router(const uint16_t* __restrict__ x,
                                                                   const uint16_t* __restrict__ wg, int H, int E,
                                                                   int k, int nb, float* logits, uint32_t* cnt,
                                                                   TopkOut o, SbParams sp) {
  static_assert(kSbRouterWaves == 1, "the shared up tiles are one-wave blocks");
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int t = blockIdx.x;
  __shared__ int last;
  if ((int)blockIdx.y >= nb) {
    __shared__ u32x4 bt[16 * 17], at[8 * 17];
    const int j = ((int)blockIdx.y - nb) * (int)gridDim.x + t, tiles = sp.I / 4;
    const int sj = j / tiles;
    if (sj < (sp.T + kSbSlice - 1) / kSbSlice) sb_shared_up<R, 4>(sp, sj, j - sj * tiles, j, bt, at);
    return;
  }
  XFrag<MAXC> xf;
  load_xfrag<MAXC>(xf, x + (size_t)t * H, H, lane);
  const int e0 = ((int)blockIdx.y * kSbRouterWaves + wid) * 4;
  float* lt = logits + (size_t)t * E;
  if (e0 < E) {
    const uint16_t* rows[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) rows[r] = wg + (size_t)min(e0 + r, E - 1) * H;
    float d[4];
    wave_dots<MAXC, 4>(rows, xf, H, lane, d);
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (e0 + r < E) __hip_atomic_store(lt + e0 + r, d[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  sb_stores_done();
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(cnt + t * kLine, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)nb - 1u;
  __syncthreads();
  if (!last) return;
  if (wid == 0) {
    o.ids32 += (size_t)t * k;
    o.wf += (size_t)t * k;
    if (o.ids64) o.ids64 += (size_t)t * k;
    if (o.wb) o.wb += (size_t)t * k;
    wave_topk<MAXEPL>(lt, true, E, k, lane, o);
    if (lane == 0) __hip_atomic_store(cnt + t * kLine, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------- host
static int sb_ring(int nkb, int rmax) {   // stages in flight: the most (<= rmax) that divide the stage count
  for (int r = rmax; r > 1; --r)
    if (nkb % r == 0) return r;
  return 1;
}

bool sb_supported(int T, int H, int I, int Is, int k, int q4) {
  if (q4 || T < 2 || T > kSbMaxTokens || T * k > kSbMaxEntries) return false;
  if (Is && Is != I) return false;
  return H % 128 == 0 && I % 128 == 0 && H / 64 <= kSbTiles;
}

static void sb_launch_up(const SbParams& p, int R, dim3 grid, hipStream_t s) {
  if (p.sh_pre) {   // R = 4 or 5 (sb_shared_pre)
    if (R == 5) hipLaunchKernelGGL((k_sb_up_shd<5>), grid, dim3(64), 0, s, p);
    else hipLaunchKernelGGL((k_sb_up_shd<4>), grid, dim3(64), 0, s, p);
    return;
  }
  switch (R) {
    case 5: hipLaunchKernelGGL((k_sb_up<5>), grid, dim3(64), 0, s, p); break;
    case 4: hipLaunchKernelGGL((k_sb_up<4>), grid, dim3(64), 0, s, p); break;
    case 3: hipLaunchKernelGGL((k_sb_up<3>), grid, dim3(64), 0, s, p); break;
    case 2: hipLaunchKernelGGL((k_sb_up<2>), grid, dim3(64), 0, s, p); break;
    default: hipLaunchKernelGGL((k_sb_up<1>), grid, dim3(64), 0, s, p); break;
  }
}

// Whether the router launch can take the shared expert's gate/up (and the up launch its down):
// a shared expert, up tiles of 4 or 5 stages in flight in the up launch and of 8 or 10 in the
// router launch, down tiles of 2, E <= 256.
static bool sb_shared_pre(bool has_sh, int H, int E, int I) {
  const int r = sb_ring(H / 128, 5), rs = sb_ring(H / 128, 10);
  return has_sh && (r == 4 || r == 5) && (rs == 8 || rs == 10) && sb_ring(I / 128, 2) == 2 && E <= 256;
}
// Token counts that take it.  Full-size layer (H=2560, E=256, I=1024, k=8, 8 rotating layers,
// same-run A/B, three rounds each): T=2 62.5-62.6 -> 60.2-60.5 us per layer; the same relocation
// at every T was slower from T=3 on (T=3 77.3 -> 77.5-77.7, T=4 94.4 -> 94.8-95.1, T=8 154.6 ->
// 156.0-156.4, T=16 259.0 -> 262.7-263.1): the shared slice is a smaller part of the up and down
// launches there, and the router launch waits for its shared tiles.  Shared tiles of 8 columns
// (5 stages in flight, four ring lengths of 80 KB) gave 61.1-61.4 at T=2 (router 7.6 -> 8.5 us);
// a delay before them made it slower still (62.1 / 62.9 / 64.6 us for ~1 / 2 / 4 us).
static bool sb_shared_pre_tokens(int T) { return T == 2; }

static SbParams sb_params(const uint16_t* x, int T, const uint16_t* sh_gate, const uint16_t* sh_up,
                          const uint16_t* sh_down, const uint16_t* sh_gate_w, int H, int E, int I, int k, int Is,
                          void* ws) {
  const Ws L = ws_layout(T, H, E, I, k, Is);
  SbParams p{};
  p.x = x;
  p.sh_gate = sh_gate; p.sh_up = sh_up; p.sh_down = sh_down; p.sh_gate_w = sh_gate_w;
  p.T = T; p.H = H; p.E = E; p.I = I; p.k = k;
  p.act = ws_ptr<uint16_t>(ws, L.act);
  p.ch = ws_ptr<uint16_t>(ws, L.ch);
  p.sh = ws_ptr<uint16_t>(ws, L.sh);
  p.gs = ws_ptr<float>(ws, L.gs);
  p.ord_row = ws_ptr<int32_t>(ws, L.sbord);
  p.ord_w = reinterpret_cast<float*>(p.ord_row + kSbMaxEntries);
  p.ord_n = p.ord_row + 2 * kSbMaxEntries;
  p.cnt = ws_ptr<uint32_t>(ws, L.sync) + kLnSbTile * kLine;
  p.slices = reinterpret_cast<SbSlice*>(p.ord_n + kSbMaxTokens);
  p.err = ws_ptr<uint32_t>(ws, L.status) + kStatusError;
  return p;
}

// Shapes must pass sb_supported; the workspace is ws_layout(T, H, E, I, k, Is).  sh_pre: the
// router launch on this stream just ran the shared expert's gate/up and gate (sb_router_launch
// reported it).
int sb_launch(const uint16_t* x, int T, const int32_t* ids32, const int64_t* ids64, const float* wf,
              const uint16_t* wb, const uint64_t* table, const uint16_t* sh_gate, const uint16_t* sh_up,
              const uint16_t* sh_down, const uint16_t* sh_gate_w, int H, int E, int I, int k, int Is,
              uint16_t* out, void* ws, hipStream_t s, const uint16_t* resid, uint32_t* err, int sh_pre) {
  const bool has_sh = sh_gate != nullptr;
  if (!has_sh) Is = 0;
  if (!sb_supported(T, H, I, Is, k, 0)) return TMOE_ERR_SHAPE;
  if (sh_pre && !sb_shared_pre(has_sh, H, E, I)) return TMOE_ERR_SHAPE;
  SbParams p = sb_params(x, T, sh_gate, sh_up, sh_down, sh_gate_w, H, E, I, k, Is, ws);
  p.ids32 = ids32; p.ids64 = ids64; p.wf = wf; p.wb = wb; p.table = table;
  p.resid = resid;
  if (err) p.err = err;
  p.out = out;
  p.sh_pre = sh_pre ? 1 : 0;
  // Slices: each group is ceil(m / 8) slices, at most T*k in all (min(E, T*k) when T <= 8).
  const int groups = E < T * k ? E : T * k;
  const int slices = T <= kSbSlice ? groups : (T * k < 2 * groups ? T * k : 2 * groups);
  const int nshs = has_sh ? (T + kSbSlice - 1) / kSbSlice : 0;
  // Up launch: the shared slices' up tiles, or with sh_pre their down tiles, then the routed
  // slices' up tiles.
  const int up_blocks = (sh_pre ? nshs * (H / 32) : nshs * (I / 8)) + slices * (I / 8);
  sb_launch_up(p, sb_ring(H / 128, 5), dim3((unsigned)up_blocks), s);
  {
    const dim3 grid((unsigned)(((sh_pre ? 0 : nshs) + slices) * (H / 32)));
    // Two stages of 32 rows in flight (deeper rings measured no faster and cost a wave slot).
    if (sb_ring(I / 128, 2) == 2) hipLaunchKernelGGL((k_sb_down<2>), grid, dim3(64), 0, s, p);
    else hipLaunchKernelGGL((k_sb_down<1>), grid, dim3(64), 0, s, p);
  }
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

// Router logits and top-k for 2 <= T <= kSbMaxTokens tokens in one launch: ids32 / wf to the
// workspace, ids64 / wb to the caller (optional), heat counters (optional).  With a shared
// expert (and shapes sb_shared_pre takes) the same launch runs the shared expert's gate/up and
// gate, and *sh_pre is set for sb_launch; the shared weights are then read while the routing
// resolves.
int sb_router_launch(const uint16_t* x, const uint16_t* wg, int T, int H, int E, int I, int k, int Is,
                     const uint16_t* sh_gate, const uint16_t* sh_up, const uint16_t* sh_gate_w, int64_t* ids64,
                     uint16_t* wb, uint32_t* heat, void* ws, hipStream_t s, int* sh_pre) {
  *sh_pre = 0;
  if (T < 1 || T > kSbMaxTokens || H % 8 || H > kMaxDim || E > kMaxExperts) return TMOE_ERR_SHAPE;
  const Ws L = ws_layout(T, H, E, I, k, Is);
  TopkOut o{};
  o.ids32 = ws_ptr<int32_t>(ws, L.ids);
  o.wf = ws_ptr<float>(ws, L.wts);
  o.ids64 = ids64;
  o.wb = wb;
  o.heat = heat;
  float* logits = ws_ptr<float>(ws, L.logits);
  uint32_t* cnt = ws_ptr<uint32_t>(ws, L.sync) + kLnSbRouter * kLine;
  const bool pre = sb_shared_pre_tokens(T) && sb_supported(T, H, I, Is, k, 0) &&
                   sb_shared_pre(sh_gate != nullptr, H, E, I);
  SbParams sp = sb_params(x, T, sh_gate, sh_up, nullptr, sh_gate_w, H, E, I, k, Is, ws);
  const int nb = (E + 4 * kSbRouterWaves - 1) / (4 * kSbRouterWaves);
  const int shared_tiles = pre ? (T + kSbSlice - 1) / kSbSlice * (I / 4) : 0;
  const dim3 g(T, nb + (shared_tiles + T - 1) / T), b(64 * kSbRouterWaves);
  const int nc = (H + 511) / 512;
  const bool r10 = sb_ring(H / 128, 10) == 10;
#define TMOE_SB_ROUTER(MAXC)                                                                                    \
  if (E > 256) hipLaunchKernelGGL((k_sb_router<MAXC, 16, 8>), g, b, 0, s, x, wg, H, E, k, nb, logits, cnt, o, sp); \
  else if (r10) hipLaunchKernelGGL((k_sb_router<MAXC, 4, 10>), g, b, 0, s, x, wg, H, E, k, nb, logits, cnt, o, sp); \
  else hipLaunchKernelGGL((k_sb_router<MAXC, 4, 8>), g, b, 0, s, x, wg, H, E, k, nb, logits, cnt, o, sp);
  switch (nc <= 2 ? 2 : nc <= 4 ? 4 : nc <= 6 ? 6 : 8) {
    case 2: TMOE_SB_ROUTER(2) break;
    case 4: TMOE_SB_ROUTER(4) break;
    case 6: TMOE_SB_ROUTER(6) break;
    default: TMOE_SB_ROUTER(8) break;
  }
#undef TMOE_SB_ROUTER
  if (hipGetLastError() != hipSuccess) return TMOE_ERR_HIP;
  *sh_pre = pre ? 1 : 0;
  return TMOE_OK;
}

}  // namespace tmoe

// Wave-level building blocks for the batch-1 (decode) path: bf16 row GEMVs with
// fp32 accumulation streamed as 16-byte loads, and the single-wave top-k.
#pragma once

#include <math.h>

#include "tmoe_device.h"
#include "tmoe_topk.h"

namespace tmoe {

// A vector of K bf16 values as seen by one wave: lane l holds columns
// c*512 + 8l .. +7 of chunk c (c < nc = ceil(K/512)), converted to fp32.
// Columns at or past K read as zero, so rows of any K % 8 == 0 work.
template <int MAXC>
struct XFrag {
  float v[MAXC][8];
};

template <int MAXC>
__device__ __forceinline__ void load_xfrag(XFrag<MAXC>& f, const uint16_t* __restrict__ x, int K, int lane) {
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int col = c * 512 + lane * 8;
    u32x4 w = {0u, 0u, 0u, 0u};
    if (col < K) w = ld16(x + col);
    f.v[c][0] = bf16_lo(w.x); f.v[c][1] = bf16_hi(w.x);
    f.v[c][2] = bf16_lo(w.y); f.v[c][3] = bf16_hi(w.y);
    f.v[c][4] = bf16_lo(w.z); f.v[c][5] = bf16_hi(w.z);
    f.v[c][6] = bf16_lo(w.w); f.v[c][7] = bf16_hi(w.w);
  }
}

// Dots of R weight rows (each K contiguous bf16) with the fragment; all R x nc
// 16-byte loads are issued before any arithmetic.  Every lane gets the sums.
template <int MAXC, int R>
__device__ __forceinline__ void wave_dots(const uint16_t* const (&rows)[R], const XFrag<MAXC>& xf, int K, int lane,
                                          float (&out)[R]) {
  u32x4 w[R][MAXC];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int col = c * 512 + lane * 8;
      w[r][c] = (col < K) ? ld_stream(rows[r] + col) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) acc = dot8(w[r][c], xf.v[c], acc);
    out[r] = wave_sum(acc);
  }
}

// The same vector kept packed (bf16 pairs): lane l holds columns c*512 + 8l .. +7
// of chunk c as 4 dwords.  EXACT: K == MAXC * 512, so no column is masked.
template <int MAXC>
struct XPack {
  u32x4 v[MAXC];
};

template <int MAXC, bool EXACT>
__device__ __forceinline__ void load_xpack(XPack<MAXC>& f, const uint16_t* __restrict__ x, int K, int lane) {
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int col = c * 512 + lane * 8;
    f.v[c] = (EXACT || col < K) ? ld16(x + col) : u32x4{0u, 0u, 0u, 0u};
  }
}

// The fragment of x = RMSNorm(h) instead (transformers modeling_qwen3_5_moe.py:806-814):
// in fp32, y = h * (1 / sqrt(mean(h^2) + eps)), then bf16(y * (1 + w)).  The squares are
// rounded and summed per lane in element order, then across the wave by an xor butterfly
// (every lane ends with the same bits), so every wave that loads it gets the same x.
template <int MAXC, bool EXACT>
__device__ __forceinline__ void load_xpack_norm(XPack<MAXC>& f, const uint16_t* __restrict__ h,
                                                const uint16_t* __restrict__ w, float eps, int K, int lane) {
  u32x4 hv[MAXC], wv[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int col = c * 512 + lane * 8;
    const bool in = EXACT || col < K;
    hv[c] = in ? ld16(h + col) : u32x4{0u, 0u, 0u, 0u};
    wv[c] = in ? ld16(w + col) : u32x4{0u, 0u, 0u, 0u};
  }
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const uint32_t q[4] = {hv[c].x, hv[c].y, hv[c].z, hv[c].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = bf16_lo(q[i]), b = bf16_hi(q[i]);
      ss = __fadd_rn(ss, __fmul_rn(a, a));
      ss = __fadd_rn(ss, __fmul_rn(b, b));
    }
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) ss = __fadd_rn(ss, __shfl_xor(ss, d));
  const float rs = 1.0f / sqrtf(__fadd_rn(ss / (float)K, eps));
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const uint32_t q[4] = {hv[c].x, hv[c].y, hv[c].z, hv[c].w};
    const uint32_t g[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = __fmul_rn(__fmul_rn(bf16_lo(q[i]), rs), __fadd_rn(1.0f, bf16_lo(g[i])));
      const float hi = __fmul_rn(__fmul_rn(bf16_hi(q[i]), rs), __fadd_rn(1.0f, bf16_hi(g[i])));
      o[i] = (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
    }
    f.v[c] = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// x, or RMSNorm(h) when a norm weight is given.
template <int MAXC, bool EXACT>
__device__ __forceinline__ void load_x(XPack<MAXC>& f, const uint16_t* x, const uint16_t* ln_w, float eps, int K,
                                       int lane) {
  if (ln_w) load_xpack_norm<MAXC, EXACT>(f, x, ln_w, eps, K, lane);
  else load_xpack<MAXC, EXACT>(f, x, K, lane);
}

// Dots of R weight rows with a packed fragment (v_dot2 bf16, fp32 accumulation);
// all R x MAXC 16-byte loads are issued before any arithmetic.  Every lane gets the sums.
template <int MAXC, int R, bool EXACT>
__device__ __forceinline__ void wave_dots_p(const uint16_t* const (&rows)[R], const XPack<MAXC>& xf, int K, int lane,
                                            float (&out)[R]) {
  u32x4 w[R][MAXC];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int col = c * 512 + lane * 8;
      w[r][c] = (EXACT || col < K) ? ld_stream(rows[r] + col) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) acc = dot8p(w[r][c], xf.v[c], acc);
    out[r] = wave_sum(acc);
  }
}

// As wave_dots_p, with the fragment produced after the weight loads are issued (get_x
// may compute it: its latency then overlaps theirs).
template <int MAXC, int R, bool EXACT, typename XGet>
__device__ __forceinline__ void wave_dots_late_x(const uint16_t* const (&rows)[R], XGet&& get_x, int K, int lane,
                                                 float (&out)[R]) {
  u32x4 w[R][MAXC];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int col = c * 512 + lane * 8;
      w[r][c] = (EXACT || col < K) ? ld_stream(rows[r] + col) : u32x4{0u, 0u, 0u, 0u};
    }
  XPack<MAXC> xf;
  get_x(xf, lane);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) acc = dot8p(w[r][c], xf.v[c], acc);
    out[r] = wave_sum(acc);
  }
}

// Top-k of E fp32 logits by one wave (lane l owns experts l + 64 i, i < MAXEPL).
// Order: logit descending, ties to the lower expert index.  Probabilities are
// softmax in fp32 (max-subtracted), renormalised over the k selected in router
// order, then rounded to bf16 -- transformers/.../modeling_qwen3_5_moe.py:771-774.
struct TopkOut {
  int32_t* ids32;    // [k] or null
  float* wf;         // [k] bf16 values as fp32, or null
  int64_t* ids64;    // [k] or null
  uint16_t* wb;      // [k] bf16 or null
  uint32_t* heat;    // [E] or null
};

// Selection and weights only, uniform across the wave (every lane holds them):
// id[r] (E for an unselectable slot) and w[r] (the bf16 weight as fp32), r < k.
struct NoPublish {
  __device__ __forceinline__ void operator()(int, int) const {}
};

// v[i] = logit of expert lane + 64 i (-inf past E).  Selection rounds run first
// (on_select(r, id) is called, wave-uniformly, as soon as slot r is known); the
// softmax denominator and the renormalised weights follow.
template <int MAXEPL, int MAXK, typename OnSelect = NoPublish>
__device__ __forceinline__ void wave_topk_values(const float (&v)[MAXEPL], int E, int k, int lane, int (&id)[MAXK],
                                                 float (&w)[MAXK], OnSelect on_select = OnSelect()) {
  uint32_t sel = 0;
  float lw[MAXK];
#pragma unroll
  for (int r = 0; r < MAXK; ++r) {
    id[r] = E;
    lw[r] = -INFINITY;
    if (r >= k) continue;                         // k is wave-uniform
    float bv = -INFINITY;
    int bi = INT_MAX;
#pragma unroll
    for (int i = 0; i < MAXEPL; ++i) {
      const int e = lane + 64 * i;
      if (e < E && !((sel >> i) & 1u) && (bi == INT_MAX || v[i] > bv)) { bv = v[i]; bi = e; }
    }
    const float g = wave_max(bv);
    const int win = wave_min_int((bi != INT_MAX && bv == g) ? bi : INT_MAX);
    if (win != INT_MAX) {
      if ((win & 63) == lane) sel |= 1u << (win >> 6);
      id[r] = win;
      lw[r] = g;
    }
    on_select(r, id[r]);
  }
  // Softmax over all E in fp32, max-subtracted (the max is the first selection).
  const float m = lw[0];
  float ls = 0.f;
#pragma unroll
  for (int i = 0; i < MAXEPL; ++i)
    if (lane + 64 * i < E) ls += expf(v[i] - m);
  const float S = wave_sum(ls);
  float p[MAXK];
  float psum = 0.f;
#pragma unroll
  for (int r = 0; r < MAXK; ++r) {
    p[r] = (r < k && id[r] != E) ? expf(lw[r] - m) / S : 0.f;
    psum += p[r];
  }
#pragma unroll
  for (int r = 0; r < MAXK; ++r) w[r] = (r < k && id[r] != E) ? rbf16(p[r] / psum) : 0.f;
}

template <int MAXEPL, int MAXK>
__device__ __forceinline__ void wave_topk_select(const float* src, int E, int k, int lane, int (&id)[MAXK],
                                                 float (&w)[MAXK]) {
  float v[MAXEPL];
#pragma unroll
  for (int i = 0; i < MAXEPL; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? src[e] : -INFINITY;
  }
  wave_topk_values<MAXEPL, MAXK>(v, E, k, lane, id, w);
}

// E <= 256 logits (4 per lane), k <= 8: the round selection of tmoe_topk.h (lane r < k
// gets slot r), then the softmax and renormalisation of wave_topk_values with the same
// operations in the same order (the denominator a wave sum, the renormalising sum over
// slots 0 .. k-1 in order), so ids and weights are bit-identical to the k-round selection;
// lane r writes slot r.
__device__ __forceinline__ void wave_topk8(const float* src, bool coherent, int E, int k, int lane,
                                           const TopkOut& o) {
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    v[i] = e >= E ? -INFINITY : coherent ? __hip_atomic_load(src + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                         : src[e];
  }
  int id = E;
  float lw = -INFINITY, top = 0.f;
  top8_rounds(v, E, k, lane, id, lw, top);
  // The largest logit (slot 0's), -inf when nothing is selectable.
  const bool any = __builtin_amdgcn_readfirstlane(id) != E;
  const float m = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(any ? lw : -INFINITY)));
  float ls = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (lane + 64 * i < E) ls += expf(v[i] - m);
  const float S = wave_sum(ls);
  const bool mine = lane < k && id != E;
  const float pr = mine ? expf(lw - m) / S : 0.f;
  float psum = 0.f;
#pragma unroll
  for (int r = 0; r < 8; ++r) psum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pr), r));
  const float w = mine ? rbf16(pr / psum) : 0.f;
  if (lane < k) {
    if (o.ids32) o.ids32[lane] = id;
    if (o.wf) o.wf[lane] = w;
    if (o.ids64) o.ids64[lane] = id;
    if (o.wb) o.wb[lane] = f32_to_bf16(w);
    if (o.heat && id < E) atomicAdd(o.heat + id, 1u);
  }
}

template <int MAXEPL>
__device__ __forceinline__ void wave_topk(const float* src, bool coherent, int E, int k, int lane, const TopkOut& o) {
  if constexpr (MAXEPL == 4) {
    if (k <= 8) return wave_topk8(src, coherent, E, k, lane, o);
  }
  int id[16];
  float w[16];
  if (coherent) {
    float v[MAXEPL];
#pragma unroll
    for (int i = 0; i < MAXEPL; ++i) {
      const int e = lane + 64 * i;
      v[i] = e < E ? __hip_atomic_load(src + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : -INFINITY;
    }
    wave_topk_values<MAXEPL, 16>(v, E, k, lane, id, w);
  } else {
    wave_topk_select<MAXEPL, 16>(src, E, k, lane, id, w);
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if (r >= k) continue;
      const int e = id[r];
      const uint16_t wb = f32_to_bf16(w[r]);
      if (o.ids32) o.ids32[r] = e;
      if (o.wf) o.wf[r] = w[r];
      if (o.ids64) o.ids64[r] = e;
      if (o.wb) o.wb[r] = wb;
      if (o.heat && e < E) atomicAdd(o.heat + e, 1u);
    }
  }
}

}  // namespace tmoe

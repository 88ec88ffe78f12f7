// Batch-1 (decode) MoE layer as ONE persistent kernel over eight dependency-ordered task queues.
//
// Tasks (each one block of 4 waves), in list order:
//   R   router rows: fp32 logits, 1 row per wave, and the shared-gate logit
//   K   gather every logit, top-k, publish the routing   (needs: all R)
//   S   shared expert gate/up pairs -> bf16 SwiGLU activations
//   SD  shared expert down, 32 rows                    (needs: the shared activations)
//   Gj  routed gate/up pairs of slot j -> activations   (needs: slot j's expert id)
//   Dj  routed down of slot j, 32 rows                  (needs: slot j's activations)
//       D(k-1), last in the list, also combines its rows from every slot's tagged
//       results: acc = bf16(acc + bf16(w_j * d_j)) in router order, then
//       acc = bf16(acc + bf16(gate * d_shared)), and writes the output.
// ordered R, K, S, SD, G0 .. G(L), then D(j-L) after each later Gj, then the
// remaining D (L = kDownLag): the shared expert streams while the router resolves,
// and a slot's down rows are drawn only once its gate/up tasks have had time to
// finish (about one resident grid of tasks later).  K publishes each expert id as
// soon as its selection round ends, so G0 starts before the top-k is complete.
//
// Hand-offs are built around two measured MI355X costs: a memory round trip under
// streaming load is ~3 us, and atomics on one hot 256-B line serialise at ~11 ns.
//   - Logits, routing and activations travel as TAGGED words: value and valid tag in
//     one device-coherent store (relaxed agent-scope atomics bypass the per-XCD L2
//     copies), so a consumer polls the data itself -- one round trip per hand-off,
//     no store-completion wait, no counter, no cache-wide write-back / invalidate.
//   - Only the row-block combine counts arrivals (one 256-B line per row block).
//   - Blocks draw tasks from eight queue counters (block b uses queue b % 8, which
//     serves tasks b % 8, +8, +16, ...).  A task only waits on tasks with smaller
//     indices and a block only draws from its own queue, so the smallest unfinished
//     task is always held, or next to be drawn, by a running block: blocks 0..7 (one
//     per queue) are dispatched first and keep drawing until their queue is empty.
//     (A cooperative launch would also guarantee residency, at ~20 us per call.)
//   - Every poll backs off exponentially and is bounded (kErrTimeout on expiry).
//   - The last combine of a call re-zeroes every tagged word and counter; the last
//     block to leave a queue re-zeroes that queue's lines.
// Reference: tarfa/engine/fused_int4.py:163-205; transformers/.../modeling_qwen3_5_moe.py:715-717, 768-798.
#include <mutex>

#include "tmoe_decode.h"
#include "tmoe_gemv.h"
#include "tmoe_ws.h"

namespace tmoe {

constexpr int kFPairsPerWave = 2;      // gate/up pairs per wave (4 rows of K = H in flight)
constexpr int kFPairsPerTask = 4 * kFPairsPerWave;
constexpr int kFDownRowsPerWave = 8;   // down rows per wave (8 rows of K = I in flight)
constexpr int kFDownRowsPerTask = 4 * kFDownRowsPerWave;
constexpr int kFusedMaxK = 8;          // top-k handled by the fused kernel (larger k takes the unfused path)
constexpr int kDownLag = 3;            // Dj is queued after G(j + kDownLag)
constexpr uint32_t kSpinLimit = 1u << 20;   // polls, each >= 64 cycles apart: never reached by a healthy graph

enum TaskType { kTR, kTK, kTS, kTSD, kTG, kTD };

__device__ __forceinline__ uint32_t ld32c(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st32c(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld64c(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st64c(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tag64(uint32_t v) { return ((uint64_t)kTag32 << 32) | v; }
__device__ __forceinline__ bool tagged64(uint64_t w) { return (uint32_t)(w >> 32) == kTag32; }
__device__ __forceinline__ uint32_t tag32(uint32_t payload16) { return (kTag16 << 16) | (payload16 & 0xFFFFu); }
__device__ __forceinline__ bool tagged32(uint32_t w) { return (w >> 16) == kTag16; }

// Every store this wave issued has completed (gfx9 counts stores in vmcnt).
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ uint32_t* line(const DecodeParams& p, int ln) { return p.sync + (size_t)ln * kLine; }

// Exponential back-off between polls; false once the bound expires (flags kErrTimeout).
struct Backoff {
  uint32_t n = 0, nap = 1;
  __device__ __forceinline__ bool step(uint32_t* err) {
    if (nap == 1) __builtin_amdgcn_s_sleep(1);
    else if (nap == 2) __builtin_amdgcn_s_sleep(2);
    else if (nap <= 4) __builtin_amdgcn_s_sleep(4);
    else if (nap <= 8) __builtin_amdgcn_s_sleep(8);
    else __builtin_amdgcn_s_sleep(16);
    nap = nap < 16 ? nap * 2 : 16;
    if (++n < kSpinLimit) return true;
    atomicOr(err, kErrTimeout);
    return false;
  }
};

// Poll one tagged 32-bit word until it is written; returns its 16-bit payload
// (or 0xFFFF after a timeout).
__device__ __forceinline__ uint32_t poll_word(const uint32_t* w, uint32_t* err) {
  Backoff b;
  for (;;) {
    const uint32_t v = ld32c(w);
    if (tagged32(v)) return v & 0xFFFFu;
    if (!b.step(err)) return 0xFFFFu;
  }
}

// A wave polls the K / 2 tagged activation pairs at w until every one it needs is
// written, and unpacks them into its fragment layout.
template <int MAXC>
__device__ __forceinline__ void poll_xfrag(XFrag<MAXC>& f, const uint64_t* w, int K, int lane, uint32_t* err) {
  Backoff b;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int col = c * 512 + lane * 8;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint64_t v = 0;
        if (col < K) {
          v = ld64c(w + col / 2 + q);
          ok = ok && tagged64(v);
        }
        f.v[c][2 * q] = bf16_lo((uint32_t)v);
        f.v[c][2 * q + 1] = bf16_hi((uint32_t)v);
      }
    }
    if (__all(ok)) return;
    if (!b.step(err)) return;
  }
}

__device__ __forceinline__ const uint32_t* route(const DecodeParams& p) {
  return line(p, kLnRoute + (int)(blockIdx.x % kRouteReplicas));
}

// Expert id of slot j for this block (thread 0 polls the routing when it comes
// from the router), broadcast through LDS; -1 for a skipped or invalid id.
__device__ __forceinline__ int block_slot_expert(const DecodeParams& p, int j, int* s_e, uint32_t* err) {
  if (threadIdx.x == 0) {
    const int e = p.ids_in ? (int)p.ids_in[j] : (int)poll_word(route(p) + kRwIds + j, err);
    if (e < 0 || e > p.E) atomicOr(err, kErrExpertId);
    *s_e = (e >= 0 && e < p.E) ? e : -1;
  }
  __syncthreads();
  return *s_e;
}

// SwiGLU of gate/up row pairs [i0, i0+2): one tagged activation pair per wave.
template <int MAXC>
__device__ __forceinline__ void up_pairs(const uint16_t* gate, const uint16_t* up, int i0, int n_rows, int K,
                                         const uint16_t* x, int lane, uint64_t* act64) {
  XFrag<MAXC> xf;
  load_xfrag<MAXC>(xf, x, K, lane);
  const uint16_t* rows[2 * kFPairsPerWave];
#pragma unroll
  for (int q = 0; q < kFPairsPerWave; ++q) {
    const int i = min(i0 + q, n_rows - 1);
    rows[q] = gate + (size_t)i * K;
    rows[kFPairsPerWave + q] = up + (size_t)i * K;
  }
  float d[2 * kFPairsPerWave];
  wave_dots<MAXC, 2 * kFPairsPerWave>(rows, xf, K, lane, d);
  static_assert(kFPairsPerWave == 2, "activations are published as one tagged bf16 pair per wave");
  if (lane == 0) {
    const uint32_t a0 = f32_to_bf16(swiglu_bf16(rbf16(d[0]), rbf16(d[2])));
    const uint32_t a1 = (i0 + 1 < n_rows) ? f32_to_bf16(swiglu_bf16(rbf16(d[1]), rbf16(d[3]))) : 0u;
    st64c(act64 + i0 / 2, tag64(a0 | (a1 << 16)));
  }
}

// 8 rows of one down projection per wave: d[r] = bf16(dot(w[h0 + r], act)).  The
// weight rows are requested before the activations are polled, so the wait for
// the producing gate/up tasks overlaps this task's own HBM traffic.
template <int MAXC>
__device__ __forceinline__ void down_dots(const uint16_t* w, const uint64_t* act64, int K, int H, int h0, int lane,
                                          float (&d)[kFDownRowsPerWave], uint32_t* err) {
  u32x4 wr[kFDownRowsPerWave][MAXC];
#pragma unroll
  for (int r = 0; r < kFDownRowsPerWave; ++r)
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int col = c * 512 + lane * 8;
      wr[r][c] = col < K ? ld_stream(w + (size_t)min(h0 + r, H - 1) * K + col) : u32x4{0u, 0u, 0u, 0u};
    }
  XFrag<MAXC> af;
  poll_xfrag<MAXC>(af, act64, K, lane, err);
#pragma unroll
  for (int r = 0; r < kFDownRowsPerWave; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) acc = dot8(wr[r][c], af.v[c], acc);
    d[r] = rbf16(wave_sum(acc));
  }
}

// Lane 0 polls the 4 tagged pairs at w until each carries `want` in its high word.
__device__ __forceinline__ void poll_pairs(const uint64_t* w, uint32_t want, uint32_t (&pair)[4], uint32_t* err) {
  Backoff b;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint64_t v = ld64c(w + q);
      ok = ok && (uint32_t)(v >> 32) == want;
      pair[q] = (uint32_t)v;
    }
    if (ok || !b.step(err)) return;
  }
}

// The K task's wave 0: gather every tagged logit, select the top-k, publish the
// routing.  Kept compact (rolled rounds, per-slot values in LDS, weights computed
// one slot per lane): this runs once per call on a cold instruction cache while
// the rest of the GPU streams, so code size is latency here.
template <int MAXEPL>
__device__ __forceinline__ void resolve_routing(const DecodeParams& p, int lane, uint32_t* err, int* s_id,
                                                float* s_lw) {
  const bool has_sh = p.sh_gate != nullptr;
  __builtin_amdgcn_s_setprio(3);   // the routing gates every expert task: issue ahead of streaming waves
  float v[MAXEPL];
  float gl = 0.f;
  Backoff b;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < MAXEPL; ++i) {
      const int e = lane + 64 * i;
      v[i] = -INFINITY;
      if (e < p.E) {
        if (p.logits_in) {
          v[i] = p.logits_in[e];
        } else {
          const uint64_t w = ld64c(p.lg64 + e);
          ok = ok && tagged64(w);
          v[i] = __uint_as_float((uint32_t)w);
        }
      }
    }
    if (has_sh) {
      const uint64_t w = ld64c(p.lg64 + p.E);
      ok = ok && tagged64(w);
      gl = __uint_as_float((uint32_t)w);
    }
    if (__all(ok)) break;
    if (!b.step(err)) break;
  }
  // Selection rounds: logit descending, ties to the lower expert index.  Each id is
  // published the moment its round ends, so slot 0's gate/up work starts at once.
  uint32_t* rep = line(p, kLnRoute + (lane & (kRouteReplicas - 1)));
  uint32_t sel = 0;
#pragma unroll 1
  for (int r = 0; r < p.k; ++r) {
    float bv = -INFINITY;
    int bi = INT_MAX;
#pragma unroll
    for (int i = 0; i < MAXEPL; ++i) {
      const int e = lane + 64 * i;
      if (e < p.E && !((sel >> i) & 1u) && (bi == INT_MAX || v[i] > bv)) {
        bv = v[i];
        bi = e;
      }
    }
    const float g = wave_max(bv);
    const int win = wave_min_int((bi != INT_MAX && bv == g) ? bi : INT_MAX);
    const int e = win == INT_MAX ? p.E : win;
    if (win != INT_MAX && (win & 63) == lane) sel |= 1u << (win >> 6);
    if (lane < kRouteReplicas) st32c(rep + kRwIds + r, tag32((uint32_t)e));
    if (lane == 0) {
      s_id[r] = e;
      s_lw[r] = g;
    }
  }
  // Softmax over all E in fp32 (max-subtracted; the max is slot 0), renormalised
  // over the k selected, rounded to bf16 -- one slot per lane.
  const float m = s_lw[0];
  float ls = 0.f;
#pragma unroll
  for (int i = 0; i < MAXEPL; ++i)
    if (lane + 64 * i < p.E) ls += expf(v[i] - m);
  const float S = wave_sum(ls);
  const bool mine = lane < p.k;
  const int id = mine ? s_id[lane] : p.E;
  const float pr = (mine && id < p.E) ? expf(s_lw[lane] - m) / S : 0.f;
  const float psum = wave_sum(pr);   // all lanes active: a DPP reduction must not run divergent
  const float wr = (mine && id < p.E) ? rbf16(pr / psum) : 0.f;
  if (mine) {
    const uint32_t tw = tag32(f32_to_bf16(wr));
#pragma unroll 1
    for (int rr = 0; rr < kRouteReplicas; ++rr) st32c(line(p, kLnRoute + rr) + kRwW + lane, tw);
    if (p.ids_out) p.ids_out[lane] = id;
    if (p.w_out) p.w_out[lane] = f32_to_bf16(wr);
    if (p.heat && id < p.E) atomicAdd(p.heat + id, 1u);
  }
  if (lane < kRouteReplicas) st32c(rep + kRwGate, tag32(has_sh ? f32_to_bf16(sigmoid_f32(rbf16(gl))) : 0u));
  if (p.logits_out)
#pragma unroll
    for (int i = 0; i < MAXEPL; ++i)
      if (lane + 64 * i < p.E) p.logits_out[lane + 64 * i] = v[i];
  __builtin_amdgcn_s_setprio(0);
}

template <int MH>
__device__ __forceinline__ void task_router(const DecodeParams& p, int t, int lane, int wid, uint32_t* err) {
  const int n_lrows = p.logits_in ? 0 : p.E;
  const int n_rows = n_lrows + (p.sh_gate ? 1 : 0);
  const int row = t * 4 + wid;
  if (row < n_rows) {
    XFrag<MH> xf;
    load_xfrag<MH>(xf, p.x, p.H, lane);
    const uint16_t* rp[1] = {row < n_lrows ? p.router_w + (size_t)row * p.H : p.sh_gate_w};
    float d[1];
    wave_dots<MH, 1>(rp, xf, p.H, lane, d);
    if (lane == 0) st64c(p.lg64 + (row < n_lrows ? row : p.E), tag64(__float_as_uint(d[0])));
  }
}

// Zero the tagged logits, activations and routing of this call (the per-slot down
// words are cleared by the combines that consume them).
__device__ __forceinline__ void reset_graph(const DecodeParams& p) {
  const int n = (p.E + 1) + (p.k * p.I + p.Is) / 2;
  for (int i = threadIdx.x; i < n; i += 256) st64c(p.lg64 + i, 0ull);
  const int rw = kRwW + p.k;   // route words in use per replica line
  for (int i = threadIdx.x; i < kRouteReplicas * rw; i += 256) st32c(line(p, kLnRoute + i / rw) + i % rw, 0u);
  if (threadIdx.x == 0) st32c(line(p, kLnCombined), 0u);
}

__device__ __forceinline__ uint64_t pack_pair_tagged(float a, float b) {
  return tag64((uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16));
}

// A D(k-1) wave: combine rows h0..h0+7 from every slot's tagged down results (its
// own in registers) and write the output.  One poll round covers everything: lane l
// fetches one word -- l < k: slot ids, k <= l < 2k: weights, l == 2k: shared gate,
// then 4 down pairs per earlier slot and 4 shared pairs -- the wave votes, and the
// values are gathered with readlane.  Consumed down words are cleared.
__device__ __forceinline__ void combine_rows(const DecodeParams& p, int e_last, int h0, int lane,
                                             const float (&d_last)[kFDownRowsPerWave], uint32_t* err) {
  const int k = p.k;
  const bool has_sh = p.sh_gate != nullptr;
  const int nq = 4 * (k - 1 + (has_sh ? 1 : 0));   // down pairs to fetch
  const int q0 = 2 * k + 1;                         // first down-pair lane
  const uint32_t* rt = route(p);
  uint64_t* src = nullptr;
  if (lane >= q0 && lane < q0 + nq) {
    const int i = lane - q0, j = i / 4;             // j == k - 1 stands for the shared slot k
    src = p.dq64 + ((size_t)(j == k - 1 ? k : j) * p.H + h0) / 2 + (i & 3);
  }
  uint32_t val = 0;
  Backoff b;
  for (;;) {
    bool ok = true;
    if (lane < k) {
      if (p.ids_in) {
        val = (uint32_t)p.ids_in[lane];
      } else {
        const uint32_t v = ld32c(rt + kRwIds + lane);
        ok = tagged32(v);
        val = v & 0xFFFFu;
      }
    } else if (lane < 2 * k) {
      if (p.w_in) {
        val = p.w_in[lane - k];
      } else {
        const uint32_t v = ld32c(rt + kRwW + (lane - k));
        ok = tagged32(v);
        val = v & 0xFFFFu;
      }
    } else if (lane == 2 * k) {
      if (has_sh) {
        const uint32_t v = ld32c(rt + kRwGate);
        ok = tagged32(v);
        val = v & 0xFFFFu;
      }
    } else if (src) {
      const uint64_t v = ld64c(src);
      ok = tagged64(v);
      val = (uint32_t)v;
    }
    if (__all(ok)) break;
    if (!b.step(err)) break;
  }
  if (src) st64c(src, 0ull);
  float acc[kFDownRowsPerWave] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < kFusedMaxK; ++j) {
    if (j >= k) continue;
    const int e = j == k - 1 ? e_last : __builtin_amdgcn_readlane((int)val, j);
    if (e < 0 || e >= p.E) continue;
    const float wj = bf16_to_f32((uint16_t)__builtin_amdgcn_readlane((int)val, k + j));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float d0 = d_last[2 * q], d1 = d_last[2 * q + 1];
      if (j != k - 1) {
        const uint32_t pr = (uint32_t)__builtin_amdgcn_readlane((int)val, q0 + 4 * j + q);
        d0 = bf16_lo(pr);
        d1 = bf16_hi(pr);
      }
      acc[2 * q] = rbf16(acc[2 * q] + rbf16(wj * d0));
      acc[2 * q + 1] = rbf16(acc[2 * q + 1] + rbf16(wj * d1));
    }
  }
  if (has_sh) {
    const float g = bf16_to_f32((uint16_t)__builtin_amdgcn_readlane((int)val, 2 * k));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t pr = (uint32_t)__builtin_amdgcn_readlane((int)val, q0 + 4 * (k - 1) + q);
      acc[2 * q] = rbf16(acc[2 * q] + rbf16(g * bf16_lo(pr)));
      acc[2 * q + 1] = rbf16(acc[2 * q + 1] + rbf16(g * bf16_hi(pr)));
    }
  }
  if (lane == 0) {
    uint32_t* o = reinterpret_cast<uint32_t*>(p.out + h0);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[q] = (uint32_t)f32_to_bf16(acc[2 * q]) | ((uint32_t)f32_to_bf16(acc[2 * q + 1]) << 16);
  }
}

struct TaskRef {
  int type, slot, idx;
};

__device__ __forceinline__ TaskRef decode_task(const DecodeParams& p, int t) {
  if (t < p.n_r) return {kTR, 0, t};
  t -= p.n_r;
  if (p.n_r) {
    if (t == 0) return {kTK, 0, 0};
    t -= 1;
  }
  if (t < p.n_s) return {kTS, 0, t};
  t -= p.n_s;
  if (p.sh_gate) {
    if (t < p.n_rb) return {kTSD, p.k, t};
    t -= p.n_rb;
  }
  for (int j = 0; j < p.k; ++j) {
    if (t < p.n_g) return {kTG, j, t};
    t -= p.n_g;
    if (j >= kDownLag) {
      if (t < p.n_rb) return {kTD, j - kDownLag, t};
      t -= p.n_rb;
    }
  }
  const int first = p.k > kDownLag ? p.k - kDownLag : 0;
  return {kTD, first + t / p.n_rb, t % p.n_rb};
}

template <int MH, int MI>
__global__ __launch_bounds__(256, 2) void k_decode_fused(DecodeParams p) {
  __shared__ int s_flag, s_e, s_task;
  __shared__ int s_id[kFusedMaxK];
  __shared__ float s_lw[kFusedMaxK];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  uint32_t* err = p.status + kStatusError;
  const int q = (int)(blockIdx.x % kQueues);
  uint32_t* queue = line(p, kLnQueue + q);
  uint32_t next = 0;
  if (threadIdx.x == 0) next = atomicAdd(queue, 1u);
  for (;;) {
    if (threadIdx.x == 0) s_task = q + kQueues * (int)next;
    __syncthreads();
    const int t = s_task;
    __syncthreads();
    if (t >= p.n_tasks) break;
    if (threadIdx.x == 0) next = atomicAdd(queue, 1u);      // draw the next task while this one runs
    const TaskRef tk = decode_task(p, t);
    if (tk.type == kTR) {
      task_router<MH>(p, tk.idx, lane, wid, err);
    } else if (tk.type == kTK) {
      if (wid == 0) {
        if (p.E <= 256)
          resolve_routing<4>(p, lane, err, s_id, s_lw);
        else
          resolve_routing<16>(p, lane, err, s_id, s_lw);
      }
    } else if (tk.type == kTS || tk.type == kTG) {
      // Gate/up pairs: the shared expert (S) or routed slot j (G); one call site.
      const bool shared = tk.type == kTS;
      const int e = shared ? 0 : block_slot_expert(p, tk.slot, &s_e, err);
      const int n_rows = shared ? p.Is : p.I;
      const int i0 = tk.idx * kFPairsPerTask + wid * kFPairsPerWave;
      if (e >= 0 && i0 < n_rows) {
        const uint16_t* gu = shared ? nullptr : reinterpret_cast<const uint16_t*>(p.table[2 * e]);
        const uint16_t* g = shared ? p.sh_gate : gu;
        const uint16_t* u = shared ? p.sh_up : gu + (size_t)p.I * p.H;
        up_pairs<MH>(g, u, i0, n_rows, p.H, p.x, lane,
                     p.act64 + (shared ? (size_t)p.k * p.I / 2 : (size_t)tk.slot * p.I / 2));
      }
    } else {
      // Down rows: the shared expert (SD, kept for the last fold) or routed slot j (D, folded).
      const bool shared = tk.type == kTSD;
      const int e = shared ? 0 : block_slot_expert(p, tk.slot, &s_e, err);
      const int h0 = tk.idx * kFDownRowsPerTask + wid * kFDownRowsPerWave;
      float d[kFDownRowsPerWave] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (e >= 0 && h0 < p.H) {
        const uint16_t* w = shared ? p.sh_down : reinterpret_cast<const uint16_t*>(p.table[2 * e + 1]);
        const uint64_t* a = p.act64 + (shared ? (size_t)p.k * p.I / 2 : (size_t)tk.slot * p.I / 2);
        down_dots<MI>(w, a, shared ? p.Is : p.I, p.H, h0, lane, d, err);
      }
      const bool last = !shared && tk.slot == p.k - 1;
      if (!last) {
        // Publish this slot's rows (a skipped slot publishes zeros the combine ignores).
        if (lane == 0 && h0 < p.H) {
          uint64_t* dst = p.dq64 + ((size_t)(shared ? p.k : tk.slot) * p.H + h0) / 2;
#pragma unroll
          for (int q = 0; q < 4; ++q) st64c(dst + q, pack_pair_tagged(d[2 * q], d[2 * q + 1]));
        }
      } else {
        if (h0 < p.H) combine_rows(p, e, h0, lane, d, err);
        // Every combine of the call done: clear the hand-off words for the next call.
        wait_stores();
        __syncthreads();
        if (threadIdx.x == 0)
          s_flag = __hip_atomic_fetch_add(line(p, kLnCombined), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   (uint32_t)p.n_rb - 1u;
        __syncthreads();
        if (s_flag) reset_graph(p);
      }
    }
  }
  // The last block to leave queue q re-zeroes its lines (every draw from it is done).
  if (threadIdx.x == 0) {
    const uint32_t users = (gridDim.x - (uint32_t)q + kQueues - 1) / kQueues;
    const uint32_t prev =
        __hip_atomic_fetch_add(line(p, kLnQueueExit + q), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == users - 1u) {
      st32c(queue, 0u);
      st32c(line(p, kLnQueueExit + q), 0u);
    }
  }
}

// ---------------------------------------------------------------- launch
typedef void (*FusedKernel)(DecodeParams);

static FusedKernel pick_fused(int ncH, int ncI) {
  const int mh = ncH <= 2 ? 2 : ncH <= 4 ? 4 : ncH <= 6 ? 6 : ncH <= 8 ? 8 : 0;
  const int mi = ncI <= 2 ? 2 : ncI <= 4 ? 4 : 0;
  switch (mh * 10 + mi) {
    case 22: return k_decode_fused<2, 2>;
    case 24: return k_decode_fused<2, 4>;
    case 42: return k_decode_fused<4, 2>;
    case 44: return k_decode_fused<4, 4>;
    case 62: return k_decode_fused<6, 2>;
    case 64: return k_decode_fused<6, 4>;
    case 82: return k_decode_fused<8, 2>;
    case 84: return k_decode_fused<8, 4>;
  }
  return nullptr;
}

// Blocks of a kernel that can be resident at once on the current device (cached).
static int resident_blocks(FusedKernel k) {
  static std::mutex mu;
  static struct {
    int dev;
    FusedKernel k;
    int n;
  } cache[64];
  static int used = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i)
    if (cache[i].dev == dev && cache[i].k == k) return cache[i].n;
  int cu = 0, occ = 0;
  if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(k), 256, 0) != hipSuccess)
    return 0;
  const int n = cu * (occ > 0 ? occ : 1);
  if (used < 64) cache[used++] = {dev, k, n};
  return n;
}

int decode_fused_launch(DecodeParams& p, bool run_router, hipStream_t s) {
  const bool has_sh = p.sh_gate != nullptr;
  const int ncH = (p.H + 511) / 512;
  const int ncI = ((p.I > p.Is ? p.I : p.Is) + 511) / 512;
  FusedKernel k = pick_fused(ncH, ncI);
  p.n_rb = (p.H + kFDownRowsPerTask - 1) / kFDownRowsPerTask;
  if (!k || p.n_rb > kMaxRowBlocks || p.k > kFusedMaxK || (has_sh && !run_router) || (p.I & 1) || (p.Is & 1))
    return TMOE_ERR_SHAPE;
  const int n_rows = (p.logits_in ? 0 : p.E) + (has_sh ? 1 : 0);
  p.n_r = run_router ? (n_rows > 0 ? (n_rows + 3) / 4 : 1) : 0;
  p.n_s = has_sh ? (p.Is + kFPairsPerTask - 1) / kFPairsPerTask : 0;
  p.n_g = (p.I + kFPairsPerTask - 1) / kFPairsPerTask;
  p.n_tasks = p.n_r + (p.n_r ? 1 : 0) + p.n_s + (has_sh ? p.n_rb : 0) + p.k * (p.n_g + p.n_rb);
  int grid = resident_blocks(k);
  if (grid <= 0) return TMOE_ERR_HIP;
  if (grid > p.n_tasks) grid = p.n_tasks;
  hipLaunchKernelGGL(k, dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

}  // namespace tmoe

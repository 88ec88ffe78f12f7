// Batch-1 (decode) MoE layer as ONE persistent kernel whose waves draw tasks from
// 32 dependency-ordered queues.
//
// Tasks (each one wave), in list order:
//   R   router rows: fp32 logits, 4 rows per task (row E = the shared-gate logit),
//       each written to all kLogitReplicas copies of the logits
//   S   shared expert gate/up, 2 row pairs -> 2 bf16 SwiGLU activations
//   SD  shared expert down, 8 rows                     (needs: every S)
//   Gj  routed gate/up of slot j, 2 row pairs          (needs: the routing)
//   Dj  routed down of slot j, 8 rows                  (needs: every Gj)
//       D(k-1), last in the list, also combines its rows from every slot's tagged
//       results: acc = bf16(acc + bf16(w_j * d_j)) in router order, then
//       acc = bf16(acc + bf16(gate * d_shared)), and writes the output.
// Int4 mode (labelled fast mode) changes the routed tasks only: G takes 2 row
// pairs of packed int4 rows with fp32 results and act = bf16(silu(g) * u), D takes
// 16 rows (8 when I > 1024) with fp32 results, and the combine is the fp32 sum
// y = y + w_j * d_j in router order, cast to bf16 once, plus the bf16 shared expert
// (tarfa/engine/moe_kernel.py:90-104, fused_int4.py:206-219).
// The list is ordered R, G0 .. G(L), then D(j-L) after each later Gj (L = kDownLag), S
// after G(kSharedAfter) and SD L slots later, then the remaining D: while the
// routing resolves only the router rows and the shared expert load, and down rows
// are drawn only once their gate/up tasks have had time to finish.
// The routing (top-k, softmax weights, shared gate) is resolved in every block: the
// first of its waves to need it polls the block's copy of the logits (32 copies, so
// 16 blocks read each), selects and writes the route words to LDS for the block.  A
// single resolving task would add a publish and a second poll through memory to the
// critical path.
//
// Hand-offs are built around measured MI355X costs: a memory round trip under
// streaming load is several us, atomics on one hot 256-B line serialise at ~11 ns,
// and every poll of a coherent word travels to the memory side like the weight
// stream itself, so polling must be cheap.
//   - Logits, activations and per-slot down rows travel as TAGGED 64-bit
//     words {payload, tag}: one device-coherent store (relaxed agent-scope atomics
//     bypass the per-XCD L2 copies), so a consumer checks the data itself -- no
//     store-completion wait, no cache-wide write-back / invalidate.
//     The tag is the call's epoch (a counter in the workspace, advanced when a
//     call ends), so words left by earlier calls never match and nothing is
//     cleared between calls; at the 2^32 wrap the ending wave zeroes the hand-off area.
//   - A down task reads its activations with plain loads issued together with its
//     weight rows (queued kDownLag slots after its gate/up tasks, the activations
//     are normally complete); stale words are re-polled with coherent loads.
//   - Each wave caches the routing; the block's copy in LDS is resolved once.
//   - Exact-bf16 mode: queue q (of 128) is served by wave q % 4 of the blocks b with
//     group(b) == q / 4, group(b) = (b % 8) * 4 + (b / 8) % 4 (the blocks of one XCD fall in 4
//     groups), and holds tasks q, q + 128, ...  (128 counters: 16 waves per counter line
//     instead of 64 keep the draws that the routing releases all at once from serialising on
//     32 lines.)  Int4 mode uses 32 queues, one group per XCD (group(b) = b % 8).  Every
//     ticket, a wave's first included, is drawn from the queue's counter: the first at entry
//     (its round trip overlaps the epoch load), every later one when a task starts,
//     read after the task's loads and before its stores (gfx9 counts stores in
//     vmcnt, and vector memory returns in issue order).  A queue's tasks are so
//     claimed in list order and only by running waves, and a task waits only on
//     tasks with smaller indices: the smallest unfinished task is always some running
//     wave's current task and can finish, whatever subset of the grid is resident,
//     as long as every queue has one running wave (one block of each of the 32 groups;
//     tests/test_ticket_progress.py simulates the task graph).  Int4 mode draws its tickets
//     the same way (its short tasks hide less of the draw's round trip, but static tickets
//     would need the whole grid resident).
//   - Every poll backs off and is bounded (kErrTimeout on expiry).
//   - The last wave to leave a queue re-zeroes its exit count; the last queue to
//     drain advances the epoch.
// Reference: tarfa/engine/fused_int4.py:163-205; transformers/.../modeling_qwen3_5_moe.py:715-717, 768-798.

#include <mutex>

#include "tmoe_decode.h"
#include "tmoe_gemv.h"
#include "tmoe_q4.h"
#include "tmoe_topk.h"
#include "tmoe_ws.h"

namespace tmoe {

constexpr int kWaves = 4;              // waves per block
constexpr int kRouterRows = 4;         // router rows per R task
constexpr int kPairs = 2;              // gate/up row pairs per G / S task (4 rows of K = H in flight)
constexpr int kQ4SPairs = 4;           // int4 mode: row pairs per (bf16) S task -- 8 rows in flight: the
                                       // int4 tasks leave registers for them, and half as many S tasks
                                       // finish the shared expert sooner in the routing window
constexpr int kDownRows = 8;           // down rows per D / SD task (8 rows of K = I in flight)
constexpr int kQ4Pairs = 2;            // int4: gate/up row pairs per G task (4 rows of H/2 bytes; 4 pairs
                                       // measured 28.4 against 27.7-28.0 us with drawn tickets)
// int4: down rows per D task (their scale words, rows * I / 256, fit two per lane)
constexpr int q4_down_rows(int MI) { return MI <= 2 ? 16 : 8; }
constexpr int kFusedMaxK = 8;          // top-k handled by the fused kernel (larger k takes the unfused path)
constexpr int kDownLag = 8;            // Dj is queued after G(j + kDownLag): with k <= 8, every D after every G
constexpr int kSharedAfter = 1;        // the shared gate/up tasks are queued after this slot's gate/up tasks
// The shared gate/up tasks' start delay, x 64 cycles: exact bf16 ~2 us; int4 ~3 us (int4 at the
// full-size layer: 32 -> 29.5-29.9 us, 64 -> 28.9-29.1, 100 -> 28.4-28.5, 127 -> 29.0-29.2).
template <bool Q4>
constexpr int shared_delay() { return Q4 ? 100 : 64; }
// Tickets: every one drawn from a per-queue counter, in both modes, so the call completes
// whatever subset of the grid is resident (the int4 mode's short tasks hide less of the draw's
// round trip than the exact-bf16 ones, but static tickets would need the whole grid resident).
template <bool Q4>
constexpr bool dynamic_tickets() { return true; }
constexpr int kBlocksPerCU = 2;        // resident blocks per CU (bounds the bytes in flight per XCD)
constexpr uint32_t kSpinLimit = 1u << 20;   // polls, each >= 64 cycles apart: never reached by a healthy graph
static_assert(kQueues == 32 * kWaves, "queue q is served by wave q % 4 of the blocks of group q / 4 (32 groups)");
// Queue groups of a mode: exact-bf16 32 (each XCD's blocks in 4 interleaved groups, 16 waves
// per counter line), int4 8 (one per XCD; 64 waves per line: measured 30.3 us per layer against
// 33.3 with 32 groups, its few short tasks per wave gaining more from the longer queues).
template <bool Q4>
constexpr int queue_groups() { return Q4 ? 8 : 32; }
// The block group of block b (NG groups): its XCD (b % 8), and with NG = 32 one of 4
// interleaved groups on it.
template <int NG>
__device__ __forceinline__ int block_group(uint32_t b) {
  return NG == 8 ? (int)(b % 8u) : (int)(b % 8u) * 4 + (int)((b / 8u) % 4u);
}

enum TaskType { kTR = 0, kTS = 2, kTSD = 3, kTG = 4, kTD = 5 };

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
// Two consecutive tagged words in one 16-byte vector store (p 16-byte aligned) with the
// cache policy of st64c's agent-scope store (sc1); each word carries its own tag, so the
// pair needs no atomicity.  (Issued from inline assembly, the store is not in the
// compiler's count of outstanding vector-memory operations; that can only make its later
// waits stricter.)
__device__ __forceinline__ void st128c(uint64_t* p, uint64_t a, uint64_t b) {
  const u32x4 v = {(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
  asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ uint32_t add32c(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A wave-uniform load of memory that no task writes during the call (expert
// table, caller-supplied routing): through the constant address space it is a
// scalar load, so waiting for it never waits for this wave's outstanding
// vector stores.
template <typename T>
__device__ __forceinline__ T ld_inv(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}
// fp16 value idx of p (4-byte aligned), as fp32, through a wave-uniform dword load.
__device__ __forceinline__ float ld_inv_f16(const uint16_t* p, int idx) {
  const uint32_t w = ld_inv(reinterpret_cast<const uint32_t*>(p) + (idx >> 1));
  return (float)__builtin_bit_cast(_Float16, (uint16_t)((idx & 1) ? (w >> 16) : (w & 0xFFFFu)));
}
__device__ __forceinline__ uint64_t tagged(uint32_t tag, uint32_t v) { return ((uint64_t)tag << 32) | v; }
__device__ __forceinline__ bool has_tag(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }

__device__ __forceinline__ uint32_t* line(const DecodeParams& p, int ln) { return p.sync + (size_t)ln * kLine; }
__device__ __forceinline__ uint64_t* line64(const DecodeParams& p, int ln) {
  return reinterpret_cast<uint64_t*>(line(p, ln));
}

// Back-off between polls, doubling up to s_sleep(MAXNAP); false once the bound
// expires (flags kErrTimeout).
template <int MAXNAP>
struct Backoff {
  uint32_t n = 0, nap = 1;
  __device__ __forceinline__ bool step(uint32_t* err) {
    if (nap == 1) __builtin_amdgcn_s_sleep(1);
    else if (nap == 2) __builtin_amdgcn_s_sleep(2);
    else if (nap <= 4) __builtin_amdgcn_s_sleep(4);
    else if (nap <= 8) __builtin_amdgcn_s_sleep(8);
    else __builtin_amdgcn_s_sleep(16);
    nap = nap < MAXNAP ? nap * 2 : MAXNAP;
    if (++n < kSpinLimit) return true;
    if ((threadIdx.x & 63) == 0) atomicOr(err, kErrTimeout);
    return false;
  }
};

// Read the K / 2 tagged activation pairs into a packed fragment (lane l: columns
// c*512 + 8l .. +7).  The first read is a plain load issued together with the
// caller's weight loads -- the producing gate/up tasks are normally long done,
// and through the XCD's L2 one memory fetch serves every wave of the XCD; words
// still carrying an old tag are re-read with coherent loads until they match.
template <int MAXC, bool EXACT>
__device__ __forceinline__ void load_acts(XPack<MAXC>& f, const uint64_t* w, int K, int lane, uint32_t tag,
                                          uint32_t* err) {
  {
    bool ok = true;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int col = c * 512 + lane * 8;
      u32x4 lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
      if (EXACT || col < K) {
        lo = ld16(w + col / 2);
        hi = ld16(w + col / 2 + 2);
        ok &= lo.y == tag && lo.w == tag && hi.y == tag && hi.w == tag;
      }
      f.v[c] = u32x4{lo.x, lo.z, hi.x, hi.z};
    }
    if (__all(ok)) return;
  }
  Backoff<4> b2;
  for (;;) {
    // All loads of a round issue before any is checked (addresses clamped, not skipped).
    uint64_t v[MAXC][4];
#pragma unroll
    for (int c = 0; c < MAXC; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) v[c][q] = ld64c(w + min(c * 512 + lane * 8, K - 8) / 2 + q);
    bool ok = true;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const bool in = EXACT || c * 512 + lane * 8 < K;
#pragma unroll
      for (int q = 0; q < 4; ++q) ok &= !in || has_tag(v[c][q], tag);
      f.v[c] = in ? u32x4{(uint32_t)v[c][0], (uint32_t)v[c][1], (uint32_t)v[c][2], (uint32_t)v[c][3]}
                  : u32x4{0u, 0u, 0u, 0u};
    }
    if (__all(ok)) return;
    if (!b2.step(err)) return;
  }
}

// The copy of the logits a block reads: one of kLogitReplicas (16 blocks per copy).
__device__ __forceinline__ int logit_copy(const DecodeParams& p) { return (int)(blockIdx.x % kLogitReplicas); }

// Routing as seen by one block: the route words (lane layout of RouteWord), set once
// (valid) by the block's resolving wave (poller).
struct RouteLds {
  uint32_t word[kRouteWords];
  uint32_t valid;    // the expert ids (words kRwId ..) are set
  uint32_t wvalid;   // the weights and the shared gate (words kRwW ..) are set
  uint32_t poller;
};
constexpr uint32_t kUnseenWord = 0xFFFFFFFFu;

// SwiGLU of gate/up row pairs [i0, i0 + P): P / 2 tagged activation pairs.
template <int MH, bool EXACT, int P, bool LATE_X, typename XGet, typename Take>
__device__ __forceinline__ void up_pairs(const uint16_t* gate, const uint16_t* up, int i0, int n_rows, int K,
                                         XGet&& get_x, int lane, uint64_t* act64, uint32_t tag, Take&& take) {
  static_assert(P % 2 == 0, "activations are published as tagged bf16 pairs");
  const uint16_t* rows[2 * P];
#pragma unroll
  for (int q = 0; q < P; ++q) {
    const int i = min(i0 + q, n_rows - 1);
    rows[q] = gate + (size_t)i * K;
    rows[P + q] = up + (size_t)i * K;
  }
  float d[2 * P];
  if constexpr (LATE_X) {
    wave_dots_late_x<MH, 2 * P, EXACT>(rows, get_x, K, lane, d);
  } else {
    XPack<MH> xf;
    get_x(xf, lane);
    wave_dots_p<MH, 2 * P, EXACT>(rows, xf, K, lane, d);
  }
  int pk[P / 2];
#pragma unroll
  for (int h = 0; h < P / 2; ++h) {
    const int i = i0 + 2 * h;
    const uint32_t a0 = i < n_rows ? f32_to_bf16(swiglu_bf16(rbf16(d[2 * h]), rbf16(d[P + 2 * h]))) : 0u;
    const uint32_t a1 =
        i + 1 < n_rows ? f32_to_bf16(swiglu_bf16(rbf16(d[2 * h + 1]), rbf16(d[P + 2 * h + 1]))) : 0u;
    pk[h] = (int)(a0 | (a1 << 16));
  }
  const uint32_t word = (uint32_t)spread(pk);
  take();
  if (lane < P / 2 && i0 + 2 * lane < n_rows) st64c(act64 + i0 / 2 + lane, tagged(tag, word));
}

// 8 rows of one down projection: d[r] = bf16(dot(w[h0 + r], act)).  The weight
// rows and the activations are requested together: one round trip when the
// producing gate/up tasks are done.
template <int MI, bool EXACT>
__device__ __forceinline__ void down_dots(const uint16_t* w, const uint64_t* act64, const DecodeParams& p, int K,
                                          int h0, int lane, float (&d)[kDownRows], uint32_t tag, uint32_t* err) {
  u32x4 wr[kDownRows][MI];
#pragma unroll
  for (int r = 0; r < kDownRows; ++r)
#pragma unroll
    for (int c = 0; c < MI; ++c) {
      const int col = c * 512 + lane * 8;
      wr[r][c] = (EXACT || col < K) ? ld_stream(w + (size_t)min(h0 + r, p.H - 1) * K + col)
                                    : u32x4{0u, 0u, 0u, 0u};
    }
  XPack<MI> af;
  load_acts<MI, EXACT>(af, act64, K, lane, tag, err);
#pragma unroll
  for (int r = 0; r < kDownRows; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < MI; ++c) acc = dot8p(wr[r][c], af.v[c], acc);
    d[r] = rbf16(wave_sum(acc));
  }
}

// Int4 SwiGLU of gate/up row pairs [i0, i0 + R) of one expert (packed gate_up rows
// [2I, H/2], scales [2I, H/128]): fp32 gate and up values (no rounding), then
// act = bf16(silu(g) * u) in fp32 (tarfa/engine/moe_kernel.py:100), published as R/2
// tagged bf16 pairs.  Loads in need order: input, scales, then the 2R weight rows.
// QR: the reference's own scale layout instead, one fp16 scale per row (gs [2I]): the row's
// fp32 dot is multiplied by it once, as the reference's kernel does (moe_kernel.py:62-63).
template <int MH, int R, bool QR, typename XGet, typename Take>
__device__ __forceinline__ void up_q4(const uint8_t* gq, const uint16_t* gs, int i0, int I, int H,
                                      XGet&& get_x, int lane, uint64_t* act64, uint32_t tag, Take&& take) {
  constexpr int G = 4 * MH;            // scale groups per row (H = 512 MH)
  constexpr int NW = R * G / 2;        // scale words of R rows
  static_assert(R % 2 == 0 && NW <= 128, "scale words of a block fit two per lane");
  XPack<MH> xf;
  get_x(xf, lane);
  // Scale words of the R gate rows and of the R up rows: word i of a block in lane i % 64, register i / 64
  // (QR: the 2R row scales, wave-uniform).
  uint32_t sc[2][2];
  float srow[2 * R];
  if constexpr (QR) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      srow[r] = ld_inv_f16(gs, i0 + r);
      srow[R + r] = ld_inv_f16(gs, I + i0 + r);
    }
  } else {
    const uint32_t* sg = reinterpret_cast<const uint32_t*>(gs + (size_t)i0 * G);
    const uint32_t* su = reinterpret_cast<const uint32_t*>(gs + (size_t)(I + i0) * G);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      sc[0][h] = (h * 64 < NW && lane + h * 64 < NW) ? sg[lane + h * 64] : 0u;
      sc[1][h] = (h * 64 < NW && lane + h * 64 < NW) ? su[lane + h * 64] : 0u;
    }
  }
  const size_t rowb = (size_t)H / 2;
  uint32_t w[2 * R][MH];
#pragma unroll
  for (int q = 0; q < R; ++q)
#pragma unroll
    for (int c = 0; c < MH; ++c) {
      w[q][c] = ld_stream4(gq + (size_t)(i0 + q) * rowb + c * 256 + lane * 4);
      w[R + q][c] = ld_stream4(gq + (size_t)(I + i0 + q) * rowb + c * 256 + lane * 4);
    }
  Q4Frag<MH> qx;
  q4_prepare(xf, qx);
  const uint32_t sel = q4_scale_sel(lane);
  float v[2 * R];
#pragma unroll
  for (int r = 0; r < 2 * R; ++r) {
    float a = 0.f;
#pragma unroll
    for (int c = 0; c < MH; ++c) {
      if constexpr (QR) {
        a += q4_dot8(w[r][c], qx.x[c], qx.off[c]);
      } else {
        // Words base, base + 1 (base even: G is a multiple of 4) share one register.
        const int base = ((r % R) * G + 4 * c) / 2;
        a = fmaf(q4_scale(sc[r / R][base / 64], (base % 64) + (lane >> 5), sel), q4_dot8(w[r][c], qx.x[c], qx.off[c]),
                 a);
      }
    }
    v[r] = QR ? wave_sum(a) * srow[r] : wave_sum(a);
  }
  int pk[R / 2];
#pragma unroll
  for (int h = 0; h < R / 2; ++h) {
    const uint32_t a0 = f32_to_bf16(silu_f32(v[2 * h]) * v[R + 2 * h]);
    const uint32_t a1 = f32_to_bf16(silu_f32(v[2 * h + 1]) * v[R + 2 * h + 1]);
    pk[h] = (int)(a0 | (a1 << 16));
  }
  const uint32_t word = (uint32_t)spread(pk);
  take();
  if (lane < R / 2) st64c(act64 + i0 / 2 + lane, tagged(tag, word));
}

// RQ rows of an int4 down projection (packed [H, I/2], scales [H, I/128]):
// d[r] = fp32 dot(w[h0 + r], act).  Weight rows and activations are requested
// together, as in down_dots.
template <int MI, int RQ, bool QR>
__device__ __forceinline__ void down_q4(const uint8_t* dq, const uint16_t* ds, const uint64_t* act64, int I, int h0,
                                        int lane, float (&d)[RQ], uint32_t tag, uint32_t* err) {
  constexpr int G = 4 * MI;            // scale groups per row (I = 512 MI)
  constexpr int NW = RQ * G / 2;       // scale words of the RQ rows
  static_assert(NW <= 128, "scale words fit two per lane");
  uint32_t sc[2];
  float srow[RQ];
  if constexpr (QR) {
#pragma unroll
    for (int r = 0; r < RQ; ++r) srow[r] = ld_inv_f16(ds, h0 + r);
  } else {
    const uint32_t* sp = reinterpret_cast<const uint32_t*>(ds + (size_t)h0 * G);
#pragma unroll
    for (int h = 0; h < 2; ++h) sc[h] = (h * 64 < NW && lane + h * 64 < NW) ? sp[lane + h * 64] : 0u;
  }
  const size_t rowb = (size_t)I / 2;
  uint32_t w[RQ][MI];
#pragma unroll
  for (int r = 0; r < RQ; ++r)
#pragma unroll
    for (int c = 0; c < MI; ++c) w[r][c] = ld_stream4(dq + (size_t)(h0 + r) * rowb + c * 256 + lane * 4);
  XPack<MI> af;
  load_acts<MI, true>(af, act64, I, lane, tag, err);
  Q4Frag<MI> qa;
  q4_prepare(af, qa);
  const uint32_t sel = q4_scale_sel(lane);
#pragma unroll
  for (int r = 0; r < RQ; ++r) {
    float a = 0.f;
#pragma unroll
    for (int c = 0; c < MI; ++c) {
      if constexpr (QR) {
        a += q4_dot8(w[r][c], qa.x[c], qa.off[c]);
      } else {
        const int base = (r * G + 4 * c) / 2;   // even: words base, base + 1 share one register
        a = fmaf(q4_scale(sc[base / 64], (base % 64) + (lane >> 5), sel), q4_dot8(w[r][c], qa.x[c], qa.off[c]), a);
      }
    }
    d[r] = QR ? wave_sum(a) * srow[r] : wave_sum(a);
  }
}

// A block's routing: one wave of the block gathers every tagged logit of the block's copy,
// selects the top-k, computes the softmax weights and the shared gate, and writes the
// route words to LDS for the whole block.  Every block resolves the routing itself: the
// selection is one wave's instruction latency (~1.1 us), and no further hand-off
// through memory follows it.
template <int MAXEPL>
__device__ __forceinline__ void resolve_block(const DecodeParams& p, int lane, uint32_t tag, uint32_t* err,
                                              RouteLds& L) {
  const bool has_sh = p.sh_gate != nullptr;
  __builtin_amdgcn_s_setprio(3);   // the routing gates every expert task: issue ahead of streaming waves
  const uint64_t* lg = p.lg64 + (size_t)logit_copy(p) * p.lg_stride;
  float v[MAXEPL];
  if (p.logits_in) {
#pragma unroll
    for (int i = 0; i < MAXEPL; ++i) {
      const int e = lane + 64 * i;
      v[i] = e < p.E ? p.logits_in[min(e, p.E - 1)] : -INFINITY;
    }
  }
  const uint64_t ts_entry = p.trace ? __builtin_amdgcn_s_memrealtime() : 0ull;
  uint64_t ts_ok = 0;
  uint32_t rounds = 0;
  if (!p.logits_in) {
    // Every load of a poll round is issued before any is waited for: the
    // addresses are clamped into the logit words, never skipped.  The shared-gate
    // logit is not waited for here: only the combine needs it.  (Two rounds in flight,
    // the second half a round trip behind, saw the logits later, not sooner: 6.5-7.8
    // against 5.0-5.7 us in the timeline, with two to three times the rounds.)
    Backoff<1> b;
    for (;;) {
      uint64_t w[MAXEPL];
#pragma unroll
      for (int i = 0; i < MAXEPL; ++i) w[i] = ld64c(lg + min(lane + 64 * i, p.E - 1));
      bool ok = true;
#pragma unroll
      for (int i = 0; i < MAXEPL; ++i) {
        const bool in = lane + 64 * i < p.E;
        ok &= !in || has_tag(w[i], tag);
        v[i] = in ? __uint_as_float((uint32_t)w[i]) : -INFINITY;
      }
      ++rounds;
      if (__all(ok)) break;
      if (!b.step(err)) break;
    }
    if (p.trace) ts_ok = __builtin_amdgcn_s_memrealtime();
  }
  int my_id = p.E;          // lane r < k: slot r's expert and logit
  float my_lw = -INFINITY;
  float m = 0.f;            // the largest logit (slot 0)
  if constexpr (MAXEPL == 4) {
    top8_rounds(v, p.E, p.k, lane, my_id, my_lw, m);
  } else {
    // Selection rounds: logit descending, ties to the lower expert index.  Each lane
    // first sorts its MAXEPL logits (value descending, index ascending), so a round
    // is one max over the lane heads, a ballot for the winner, and a pop.
    float a[MAXEPL];
    int ai[MAXEPL];
#pragma unroll
    for (int i = 0; i < MAXEPL; ++i) {
      a[i] = lane + 64 * i < p.E ? v[i] : -INFINITY;
      ai[i] = lane + 64 * i;
    }
#pragma unroll
    for (int x = 0; x < MAXEPL; ++x)
#pragma unroll
      for (int y = MAXEPL - 1; y > x; --y) {
        const bool sw = a[y] > a[y - 1];   // equal values keep the lower index (earlier) first
        const float fa = sw ? a[y] : a[y - 1], fb = sw ? a[y - 1] : a[y];
        const int ia = sw ? ai[y] : ai[y - 1], ib = sw ? ai[y - 1] : ai[y];
        a[y - 1] = fa; a[y] = fb; ai[y - 1] = ia; ai[y] = ib;
      }
  #pragma unroll 1
    for (int r = 0; r < p.k; ++r) {
      const float g = wave_max(a[0]);
      const uint64_t cand = __ballot(a[0] == g && a[0] != -INFINITY);
      int win;
      if (__builtin_popcountll(cand) == 1) {
        win = __builtin_amdgcn_readlane(ai[0], (int)__builtin_ctzll(cand));
      } else {
        // Equal logits in several lanes (or none left): lowest index among them.
        win = wave_min_int(a[0] == g && a[0] != -INFINITY ? ai[0] : INT_MAX);
      }
      if (win != INT_MAX && (win & 63) == lane) {
#pragma unroll
        for (int i = 0; i + 1 < MAXEPL; ++i) {
          a[i] = a[i + 1];
          ai[i] = ai[i + 1];
        }
        a[MAXEPL - 1] = -INFINITY;
      }
      if (lane == r) {
        my_id = win == INT_MAX ? p.E : win;
        my_lw = g;
      }
      if (r == 0) m = g;
    }
  }
  const uint64_t ts_sel = p.trace ? __builtin_amdgcn_s_memrealtime() : 0ull;
  // The ids go to the block at once: the expert tasks need them, the weights and the gate
  // only their combine.
  if (lane < kRwW) L.word[kRwId + lane] = (uint32_t)my_id;
  __threadfence_block();
  if (lane == 0) __hip_atomic_store(&L.valid, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  __builtin_amdgcn_s_setprio(0);
  // Softmax over all E in fp32 (max-subtracted), renormalised over the k
  // selected, rounded to bf16 -- one slot per lane.
  float ls = 0.f;
#pragma unroll
  for (int i = 0; i < MAXEPL; ++i)
    if (lane + 64 * i < p.E) ls += expf(v[i] - m);
  const float S = wave_sum(ls);
  const bool mine = lane < p.k;
  const float pr = (mine && my_id < p.E) ? expf(my_lw - m) / S : 0.f;
  const float psum = wave_sum(pr);   // all lanes active: a DPP reduction must not run divergent
  const float wr = (mine && my_id < p.E) ? rbf16(pr / psum) : 0.f;
  const uint32_t wb = f32_to_bf16(wr);
  // Route words: lanes 0..7 the ids (E for slots past k), lanes 8..15 the weights of
  // slots 0..7, lane 16 the gate.
  const uint32_t wsrc = (uint32_t)__builtin_amdgcn_ds_bpermute(((lane - kRwW) & 63) * 4, (int)wb);
  // The shared-gate logit (row E of the router tasks), polled now that the ids are out.
  float gl = 0.f;
  if (has_sh) {
    Backoff<4> b;
    for (;;) {
      const uint64_t wg = ld64c(lg + p.E);
      gl = __uint_as_float((uint32_t)wg);
      if (has_tag(wg, tag)) break;
      if (!b.step(err)) break;
    }
  }
  const uint32_t gate = has_sh ? f32_to_bf16(sigmoid_f32(rbf16(gl))) : 0u;
  const uint64_t ts_soft = p.trace ? __builtin_amdgcn_s_memrealtime() : 0ull;
  if (lane >= kRwW && lane < kRouteWords) L.word[lane] = lane < kRwGate ? wsrc : gate;
  __threadfence_block();
  if (lane == 0) __hip_atomic_store(&L.wvalid, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  if (p.trace && lane == 0) {
    uint64_t* rec = p.trace + kTraceHeader + (size_t)p.n_tasks * kTraceTaskWords + 2 * (size_t)gridDim.x * 4 +
                    8 * (size_t)blockIdx.x;
    rec[0] = ts_entry;
    rec[1] = ts_ok;
    rec[2] = __builtin_amdgcn_s_memrealtime();
    rec[3] = rounds;
    rec[4] = ts_sel;
    rec[5] = ts_soft;
  }
}

// The wave's routing cache `rwc` (lane l < kRouteWords holds route word l) from the
// block's copy in LDS, resolved first by whichever wave of the block gets there first.
__device__ __forceinline__ void route_fetch(const DecodeParams& p, int lane, uint32_t& rwc, uint32_t tag,
                                           uint32_t* err, RouteLds& L) {
  Backoff<16> b;
  for (;;) {
    if (__hip_atomic_load(&L.valid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) break;
    uint32_t got = 0;
    if (lane == 0) got = atomicCAS(&L.poller, 0u, 1u) == 0u;
    if (__builtin_amdgcn_readfirstlane(got)) {
      if (p.E <= 256)
        resolve_block<4>(p, lane, tag, err, L);
      else
        resolve_block<16>(p, lane, tag, err, L);
      break;
    }
    if (!b.step(err)) break;
  }
  __threadfence_block();
  if (lane < kRwW) rwc = L.word[kRwId + lane];
}

// The routing weights and the shared gate into the wave's cache (lanes kRwW ..): set by the
// block's resolving wave right after the ids, long before any combine asks for them.
__device__ __forceinline__ void route_weights(int lane, uint32_t& rwc, uint32_t* err, RouteLds& L) {
  Backoff<16> b;
  while (!__hip_atomic_load(&L.wvalid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP))
    if (!b.step(err)) break;
  __threadfence_block();
  if (lane >= kRwW && lane < kRouteWords) rwc = L.word[lane];
}

// The call's routing outputs (ids, bf16 weights, heat counts, logits), written once: by
// the wave that runs the first gate/up task.
__device__ __forceinline__ void publish_routing(const DecodeParams& p, int lane, uint32_t rwc) {
  const uint32_t wv = (uint32_t)__builtin_amdgcn_ds_bpermute(((kRwW + lane) & 63) * 4, (int)rwc);
  if (lane < p.k) {
    if (p.ids_out) p.ids_out[lane] = (int64_t)rwc;
    if (p.w_out) p.w_out[lane] = (uint16_t)wv;
    if (p.heat && rwc < (uint32_t)p.E) atomicAdd(p.heat + rwc, 1u);
  }
  if (p.logits_out) {
    const uint64_t* lg = p.lg64 + (size_t)logit_copy(p) * p.lg_stride;
    for (int e = lane; e < p.E; e += 64)
      p.logits_out[e] = p.logits_in ? p.logits_in[e] : __uint_as_float((uint32_t)ld64c(lg + e));
  }
}

// Expert of slot j (wave-uniform) for this wave, or -1 for a skipped or invalid id.
__device__ __forceinline__ int wave_slot_expert(const DecodeParams& p, int j, uint32_t rwc) {
  const uint32_t w = (uint32_t)__builtin_amdgcn_readlane((int)rwc, kRwId + j);
  return (w != kUnseenWord && (int)w < p.E) ? (int)w : -1;
}

// Router rows [4t, 4t + 4) of E + 1 (row E: the shared-gate weight).
// LATE_X: the input is produced after the rows' loads are issued (a wave's first router
// task forms the normalised input then, overlapping the rows' latency).
template <int MH, bool EXACT, bool LATE_X, typename XGet, typename Take>
__device__ __forceinline__ void task_router(const DecodeParams& p, int t, int lane, XGet&& get_x, uint32_t tag,
                                            Take&& take) {
  const int n_lrows = p.logits_in ? 0 : p.E;
  const int n_rows = n_lrows + (p.sh_gate ? 1 : 0);
  const int r0 = t * kRouterRows;
  if (r0 >= n_rows) return;
  float d[kRouterRows];
  if constexpr (LATE_X) {
    const uint16_t* rp[kRouterRows];
#pragma unroll
    for (int r = 0; r < kRouterRows; ++r) {
      const int row = min(r0 + r, n_rows - 1);
      rp[r] = row < n_lrows ? p.router_w + (size_t)row * p.H : p.sh_gate_w;
    }
    wave_dots_late_x<MH, kRouterRows, EXACT>(rp, get_x, p.H, lane, d);
  } else {
    XPack<MH> xf;
    get_x(xf, lane);
    const uint16_t* rp[kRouterRows];
#pragma unroll
    for (int r = 0; r < kRouterRows; ++r) {
      const int row = min(r0 + r, n_rows - 1);
      rp[r] = row < n_lrows ? p.router_w + (size_t)row * p.H : p.sh_gate_w;
    }
    wave_dots_p<MH, kRouterRows, EXACT>(rp, xf, p.H, lane, d);
  }
  take();
  // One store instruction: lane l writes rows 2 (l % 2) and 2 (l % 2) + 1 of copy l / 2 as
  // one 16-byte store of two tagged words (the task's rows are consecutive logit indices,
  // E - 1 and E included; the shared-gate row alone, with logits supplied, is one word).
  static_assert(kRouterRows == 4 && kLogitReplicas == 32, "4 rows x 32 copies in one store instruction");
  const int ra = r0 + 2 * (lane & 1), rb = ra + 1;
  const size_t ia = ra < n_lrows ? (size_t)ra : (size_t)p.E;
  const uint32_t va = __float_as_uint((lane & 1) ? d[2] : d[0]);
  const uint32_t vb = __float_as_uint((lane & 1) ? d[3] : d[1]);
  uint64_t* dst = p.lg64 + (size_t)(lane >> 1) * p.lg_stride + ia;
  if (rb < n_rows && ia + 1 == (rb < n_lrows ? (size_t)rb : (size_t)p.E)) {
    st128c(dst, tagged(tag, va), tagged(tag, vb));
  } else if (ra < n_rows) {
    st64c(dst, tagged(tag, va));
    if (rb < n_rows) st64c(p.lg64 + (size_t)(lane >> 1) * p.lg_stride + (rb < n_lrows ? (size_t)rb : (size_t)p.E),
                           tagged(tag, vb));
  }
}

// The words a D(k-1) task combines (lane r < 8: its row h0 + r of each earlier slot, then
// of the shared expert; clamped addresses), one batch of loads after the task's own rows.
// (Requested before the rows, to overlap the round trip, they cost the exact-bf16 call
// 0.2-0.5 us in a same-run A/B, and between the rows and the activations 0.3-0.8 us, while
// the int4 mode, whose down tasks are shorter, gains 0.8 us that way: combine_words_q4.)
__device__ __forceinline__ void combine_words(const DecodeParams& p, int h0, int lane, uint64_t (&v)[kFusedMaxK]) {
  const int r = lane & (kDownRows - 1);
#pragma unroll
  for (int j = 0; j < kFusedMaxK; ++j) {
    const int slot = j < p.k - 1 ? j : p.k;
    v[j] = ld64c(p.dq64 + ((size_t)slot * p.H + h0 + r) / 2);
  }
}

// A D(k-1) task: combine rows h0..h0+7 from every slot's tagged down results (its
// own in registers) and write the output.  The routing comes from the wave's
// cache.  Lane r < 8 owns row h0 + r: it checks the words of combine_words (pre),
// re-reading them while any still carries an old tag, then folds in router order,
// acc = bf16(acc + bf16(w_j * d_j)), and adds bf16(gate * d_shared).
__device__ __forceinline__ void combine_rows(const DecodeParams& p, int e_last, int h0, int lane,
                                             const float (&d_last)[kDownRows], uint32_t& rwc, uint32_t tag,
                                             uint32_t* err, RouteLds& L, const uint64_t (&pre)[kFusedMaxK]) {
  const int k = p.k;
  const bool has_sh = p.sh_gate != nullptr;
  const int r = lane & (kDownRows - 1);
  // The residual row (layer mode), requested before the wait for the other slots.
  const float hres = p.resid ? bf16_to_f32(p.resid[h0 + r]) : 0.f;
  // Word j holds this lane's row of slot j (j < k - 1) or, at j = k - 1, of the
  // shared expert (slot k); words past that are never used.
  uint32_t pr[kFusedMaxK];
  Backoff<4> b;
  uint64_t v[kFusedMaxK];
#pragma unroll
  for (int j = 0; j < kFusedMaxK; ++j) v[j] = pre[j];
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < kFusedMaxK; ++j) {
      const bool used = j < k - 1 || (j == k - 1 && has_sh);
      ok &= !used || has_tag(v[j], tag);
      pr[j] = (uint32_t)v[j];
    }
    if (__all(ok)) break;
    if (!b.step(err)) break;
    combine_words(p, h0, lane, v);
  }
  // Lane r < 8 takes its own row of this slot (the row values are wave-uniform).
  static_assert(kDownRows == 8, "one row per lane of lanes 0..7");
  int rows[kDownRows];
#pragma unroll
  for (int i = 0; i < kDownRows; ++i) rows[i] = __float_as_int(d_last[i]);
  const float own = __int_as_float(spread8(rows));
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < kFusedMaxK; ++j) {
    if (j >= k) break;
    const uint32_t rid = (uint32_t)__builtin_amdgcn_readlane((int)rwc, kRwId + j);
    const uint32_t rwt = (uint32_t)__builtin_amdgcn_readlane((int)rwc, kRwW + j);
    const int e = j == k - 1 ? e_last : (rid == kUnseenWord ? -1 : (int)rid);
    if (e < 0 || e >= p.E || rwt == kUnseenWord) continue;
    const float wj = bf16_to_f32((uint16_t)rwt);
    const float d = j == k - 1 ? own : ((r & 1) ? bf16_hi(pr[j]) : bf16_lo(pr[j]));
    acc = rbf16(acc + rbf16(wj * d));
  }
  if (has_sh) {
    const float g = bf16_to_f32((uint16_t)__builtin_amdgcn_readlane((int)rwc, kRwGate));
    uint32_t ps = pr[0];
#pragma unroll
    for (int j = 1; j < kFusedMaxK; ++j) ps = j == k - 1 ? pr[j] : ps;
    acc = rbf16(acc + rbf16(g * ((r & 1) ? bf16_hi(ps) : bf16_lo(ps))));
  }
  if (p.resid) acc = hres + acc;   // the layer's residual add
  if (lane < kDownRows) p.out[h0 + lane] = f32_to_bf16(acc);
}

// Int4 mode: the words the last slot's task combines, one fp32 row per word, requested
// before the task's own rows and scales: the other slots' down tasks for these rows were
// queued long before, so the words have usually landed when the combine reads them and it
// costs no round trip of its own at the end of the call (30.4-30.6 -> 29.5-29.9 us).
template <int RQ>
__device__ __forceinline__ void combine_words_q4(const DecodeParams& p, int h0, int lane, uint64_t (&v)[kFusedMaxK]) {
  const int r = lane & (RQ - 1);
#pragma unroll
  for (int j = 0; j < kFusedMaxK; ++j) {
    const int slot = j < p.k - 1 ? j : p.k;
    v[j] = ld64c(p.dq64 + (size_t)slot * p.H + h0 + r);
  }
}
// Int4 mode: the combine of rows h0 .. h0 + RQ - 1 (lane r < RQ owns row h0 + r).
// Each slot's fp32 row is weighted and summed in fp32 in router order,
// y = y + w_j * d_j with separately rounded products and sums (the reference's
// fp32 weighted sum, tarfa/engine/moe_kernel.py:103), cast to bf16 once (:104);
// then the block adds the bf16 shared expert, bf16(y + bf16(gate * d_shared)).
template <int RQ>
__device__ __forceinline__ void combine_q4(const DecodeParams& p, int e_last, int h0, int lane,
                                           const float (&d_last)[RQ], uint32_t& rwc, uint32_t tag, uint32_t* err,
                                           RouteLds& L, const uint64_t (&pre)[kFusedMaxK]) {
  const int k = p.k;
  const bool has_sh = p.sh_gate != nullptr;
  const int r = lane & (RQ - 1);
  // The residual row (layer mode), requested before the wait for the other slots.
  const float hres = p.resid ? bf16_to_f32(p.resid[h0 + r]) : 0.f;
  uint32_t pr[kFusedMaxK];   // word j: this lane's row of slot j (j < k - 1) or of the shared expert (j = k - 1)
  Backoff<4> b;
  uint64_t v[kFusedMaxK];
#pragma unroll
  for (int j = 0; j < kFusedMaxK; ++j) v[j] = pre[j];
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < kFusedMaxK; ++j) {
      const bool used = j < k - 1 || (j == k - 1 && has_sh);
      ok &= !used || has_tag(v[j], tag);
      pr[j] = (uint32_t)v[j];
    }
    if (__all(ok)) break;
    if (!b.step(err)) break;
    combine_words_q4<RQ>(p, h0, lane, v);
  }
  int rows[RQ];
#pragma unroll
  for (int i = 0; i < RQ; ++i) rows[i] = __float_as_int(d_last[i]);
  const float own = __int_as_float(spread(rows));
  float y = 0.f;
#pragma unroll
  for (int j = 0; j < kFusedMaxK; ++j) {
    if (j >= k) break;
    const uint32_t rid = (uint32_t)__builtin_amdgcn_readlane((int)rwc, kRwId + j);
    const uint32_t rwt = (uint32_t)__builtin_amdgcn_readlane((int)rwc, kRwW + j);
    const int e = j == k - 1 ? e_last : (rid == kUnseenWord ? -1 : (int)rid);
    if (e < 0 || e >= p.E || rwt == kUnseenWord) continue;
    const float d = j == k - 1 ? own : __uint_as_float(pr[j]);
    y = __fadd_rn(y, __fmul_rn(d, bf16_to_f32((uint16_t)rwt)));
  }
  float acc = rbf16(y);
  if (has_sh) {
    const float g = bf16_to_f32((uint16_t)__builtin_amdgcn_readlane((int)rwc, kRwGate));
    uint32_t ps = pr[0];
#pragma unroll
    for (int j = 1; j < kFusedMaxK; ++j) ps = j == k - 1 ? pr[j] : ps;
    acc = rbf16(acc + rbf16(g * __uint_as_float(ps)));
  }
  if (p.resid) acc = hres + acc;   // the layer's residual add
  if (lane < RQ) p.out[h0 + lane] = f32_to_bf16(acc);
}

// Int4 mode, a D task of routed slot j: RQ rows published as one fp32 word each (a
// skipped slot publishes zeros the combine ignores), or combined for the last slot.
template <int MI, int RQ, bool QR, typename Take>
__device__ __forceinline__ void task_down_q4(const DecodeParams& p, int slot, int idx, int lane, uint32_t& rwc,
                                             uint32_t tag, uint32_t* err, RouteLds& L, Take&& take) {
  const int e = wave_slot_expert(p, slot, rwc);
  const int h0 = idx * RQ;
  float d[RQ];
#pragma unroll
  for (int r = 0; r < RQ; ++r) d[r] = 0.f;
  uint64_t pre[kFusedMaxK];   // the last slot's combine words, requested before the rows (see combine_words)
  if (slot == p.k - 1) combine_words_q4<RQ>(p, h0, lane, pre);
  if (e >= 0)
    down_q4<MI, RQ, QR>(reinterpret_cast<const uint8_t*>(ld_inv(p.table + 4 * e + 2)),
                    reinterpret_cast<const uint16_t*>(ld_inv(p.table + 4 * e + 3)), p.act64 + (size_t)slot * p.I / 2,
                    p.I, h0, lane, d, tag, err);
  if (e >= 0) take();
  if (slot != p.k - 1) {
    int rows[RQ];
#pragma unroll
    for (int r = 0; r < RQ; ++r) rows[r] = __float_as_int(d[r]);
    const int row = spread(rows);
    if (lane < RQ) st64c(p.dq64 + (size_t)slot * p.H + h0 + lane, tagged(tag, (uint32_t)row));
  } else {
    combine_q4<RQ>(p, e, h0, lane, d, rwc, tag, err, L, pre);
  }
}

struct TaskRef {
  int type, slot, idx;
};



// Task t of the list R, then per slot j: Gj, D(j - kDownLag) once j >= kDownLag,
// S after G(sh_after) (right after R when sh_after < 0) and SD after G(sd_after); then the
// remaining D.  Pure arithmetic on values held in scalar registers: a lookup table in
// kernel-argument memory costs a memory round trip per step.
__device__ __forceinline__ TaskRef decode_task(const DecodeParams& p, int t) {
  if (t < p.n_r) return {kTR, 0, t};
  t -= p.n_r;
  if (p.sh_after < 0) {
    if (t < p.n_s) return {kTS, 0, t};
    t -= p.n_s;
  }
  for (int j = 0; j < p.k; ++j) {
    if (t < p.n_g) return {kTG, j, t};
    t -= p.n_g;
    if (j >= kDownLag) {
      if (t < p.n_d) return {kTD, j - kDownLag, t};
      t -= p.n_d;
    }
    if (j == p.sh_after) {
      if (t < p.n_s) return {kTS, 0, t};
      t -= p.n_s;
    }
    if (j == p.sd_after) {
      if (t < p.n_sd) return {kTSD, p.k, t};
      t -= p.n_sd;
    }
  }
  const int first = p.k > kDownLag ? p.k - kDownLag : 0;
  return {kTD, first + t / p.n_d, t % p.n_d};
}

// The call is over (every queue drained): advance the epoch.  At the wrap the hand-off area is zeroed first, so tags
// restart at 1 with no stale match.
__device__ __forceinline__ void finish_call(const DecodeParams& p, uint32_t tag, int lane) {
  const bool wrap = tag == 0xFFFFFFFFu;
  if (wrap) {
    uint64_t* w = reinterpret_cast<uint64_t*>(p.handoff);
    for (size_t i = lane; i < p.handoff_words; i += 64) st64c(w + i, 0ull);
  }
  const uint32_t epoch = wrap ? 0u : tag;
  for (int j = lane; j < kQueues; j += 64) st32c(line(p, kLnQueue + j) + kQueueEpochWord, epoch);
  if (lane == 0) {
    st32c(line(p, kLnQueuesDone), 0u);
    st32c(line(p, kLnEpoch), epoch);
  }
}

// Q4: routed experts in int4 (table [E][4]); the shared expert stays bf16.  LN: the input
// is the hidden state before the layer's RMSNorm (every task that loads x forms it) and
// the combine adds the residual; without LN both pointers are null constants here, so
// none of that code is in the kernel.
// TRACE: the debug-timeline instantiation (exact-fit block shapes only); without it the
// pointer is a null constant and no recording code or state is in the kernel.
template <int MH, int MI, bool EXACT, bool Q4, bool LN, bool TRACE = false, bool QR = false>
__global__ __launch_bounds__(256, 2) void k_decode_fused(DecodeParams p) {
  static_assert(!QR || Q4, "per-row scales are an int4 format");
  static_assert(!Q4 || EXACT, "int4 variants need H and I multiples of 512");
  if constexpr (!LN) {
    p.ln_w = nullptr;
    p.resid = nullptr;
  }
  if constexpr (!TRACE) p.trace = nullptr;
  constexpr int RQ = q4_down_rows(MI);
  const int lane0 = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint32_t* err = p.err;
  {
    // Bring every 64-byte line of the kernel arguments into the scalar cache in one round
    // trip: the compiler reads fields where it first needs them, and a field on a line not
    // yet cached costs a memory round trip of its own before the first task can start.
    typedef const __attribute__((address_space(4))) uint32_t ka_u32;
    ka_u32* ka = (ka_u32*)__builtin_amdgcn_kernarg_segment_ptr();
    uint32_t touch = 0;
#pragma unroll
    for (int o = 0; o < (int)(sizeof(DecodeParams) / 4); o += 16) touch ^= ka[o];
    if (touch == 0x9E3779B9u && threadIdx.x == 0x3FF) err = nullptr;   // never taken: only makes the loads needed
  }
  constexpr int NG = queue_groups<Q4>();
  constexpr int NQ = NG * kWaves;            // queues of this mode (the first NQ of kQueues)
  const int grp = block_group<NG>(blockIdx.x);
  const int q = grp * kWaves + wid;
  uint32_t* queue = line(p, kLnQueue + q);
  // Blocks of this group: b = g0 + NG r, r = 0, 1, ... (g0 = x + 8 g for group 4 x + g of 32).
  const uint32_t g0 = NG == 8 ? (uint32_t)grp : (uint32_t)(grp / 4 + 8 * (grp % 4));
  const uint32_t users = (gridDim.x - g0 + NG - 1u) / (uint32_t)NG;
  const uint32_t rank = blockIdx.x / (uint32_t)NG;
  constexpr bool DYN = dynamic_tickets<Q4>();
  uint32_t* draw = line(p, kLnQueueExit + q) + kQueueDrawWord;
  // Exact-bf16 mode: the first ticket, drawn at once; read where the first task starts.
  uint32_t first = 0;
  if (DYN && lane0 == 0) {
    uintptr_t a = reinterpret_cast<uintptr_t>(draw);
    asm volatile("" : "+v"(a));
    first = __hip_atomic_fetch_add(reinterpret_cast<__attribute__((address_space(1))) uint32_t*>(a), 1u,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // Every lane loads the epoch (one transaction); kept per lane, the value is
  // first waited for where a task stores or polls.
  const uint32_t tag = ld32c(queue + kQueueEpochWord) + 1u;
  __shared__ RouteLds s_rt;     // the block's view of the routing
  // LN: the block's normalised input, formed by one of its waves (s_xstate 0 -> 1 claimed -> 2
  // published in s_x); the others copy it.
  __shared__ u32x4 s_x[LN ? MH * 64 : 1];
  __shared__ uint32_t s_xstate;
  if (threadIdx.x == 0) {
    s_rt.valid = 0u;
    s_rt.wvalid = 0u;
    s_rt.poller = 0u;
    s_xstate = 0u;
  }
  __syncthreads();

  uint32_t rwc = kUnseenWord;   // this wave's routing cache (lane layout of RouteWord)
  bool routed = p.ids_in != nullptr;
  bool weighted = p.ids_in != nullptr;   // rwc holds the weights and the gate too
  if (p.ids_in) {
    // Caller-supplied routing (ids outside [0, E) are skipped; E is the sentinel).
    if (lane0 < p.k) {
      const int64_t e = p.ids_in[lane0];
      rwc = e >= 0 && e < p.E ? (uint32_t)e : 0xFFFFu;
      if ((e < 0 || e > p.E) && blockIdx.x == 0 && wid == 0) atomicOr(err, kErrExpertId);
    } else if (lane0 >= kRwW && lane0 < kRwW + p.k) {
      rwc = p.w_in[lane0 - kRwW];
    }
  }
  // The input fragment: loaded per task; with LN formed once per wave (the norm needs a
  // wave reduction over h) and kept in registers for the wave's later tasks.
  XPack<MH> xcache;
  bool have_x = false;
  // LN: the first wave of the block to claim the input forms it and publishes it in LDS; a wave
  // that finds it claimed copies it once published (the claimer's loads and norm are bounded).
  // One norm per block instead of per wave: 2048 waves each reading h and the norm weight at
  // entry queued the router rows' loads behind 20 MB of requests (router loads 3.3 -> 1.4 us,
  // routing resolved 10.0 -> 8.7 us in the per-task timeline; layer 36.2-36.8 -> 36.1-36.5 us).
  // Only lane 0 takes part in the claim.
  auto claim_x = [&](int lane) {
    uint32_t st = 0;
    if (lane == 0) st = atomicCAS(&s_xstate, 0u, 1u);
    return __builtin_amdgcn_readfirstlane((int)st) == 0;
  };
  auto form_x = [&](int lane) {
    load_xpack_norm<MH, EXACT>(xcache, p.x, p.ln_w, p.ln_eps, p.H, lane);
#pragma unroll
    for (int c = 0; c < MH; ++c) s_x[c * 64 + lane] = xcache.v[c];
    __hip_atomic_store(&s_xstate, 2u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  auto get_x = [&](XPack<MH>& xf, int lane) {
    if constexpr (LN) {
      if (!have_x) {
        if (claim_x(lane)) {
          form_x(lane);
        } else {
          Backoff<4> b;
          while (__hip_atomic_load(&s_xstate, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != 2u)
            if (!b.step(err)) break;
#pragma unroll
          for (int c = 0; c < MH; ++c) xcache.v[c] = s_x[c * 64 + lane];
        }
        have_x = true;
      }
      xf = xcache;
    } else {
      load_xpack<MH, EXACT>(xf, p.x, p.H, lane);
    }
  };
  uint32_t ticket = DYN ? (uint32_t)__builtin_amdgcn_readlane((int)first, 0) : rank;
  // Waves whose first task (the drawn ticket's) is not a router task form x at once: most of
  // them next wait for the routing, which this overlaps (router waves form it inside their
  // task instead, behind their rows' loads).  Deciding by the block's rank instead, as with
  // static tickets, left the waves that drew another wave's planned router task to form x on
  // first use: 39.1-39.2 against 37.9-38.2 us per layer.
  if constexpr (LN) {
    if (q + NQ * (int)ticket >= p.n_r && claim_x(lane0)) {
      form_x(lane0);
      have_x = true;
    }
  }
  const uint64_t t_entry = p.trace ? __builtin_amdgcn_s_memrealtime() : 0ull;
  if (p.trace && blockIdx.x == 0 && wid == 0 && lane0 == 0) {
    const uint64_t hdr[kTraceHeader] = {(uint64_t)p.n_tasks, gridDim.x, (uint64_t)p.n_r, (uint64_t)p.n_s,
                                        (uint64_t)p.n_sd, (uint64_t)p.n_g, (uint64_t)p.n_d, (uint64_t)p.k,
                                        (uint64_t)p.sh_after, (uint64_t)p.sd_after, (uint64_t)kDownLag,
                                        (uint64_t)p.q4, 0, 0, 0, 0};
    for (int i = 0; i < kTraceHeader; ++i) p.trace[i] = hdr[i];
  }
  for (uint32_t i = 0;; ++i) {
    const int t = q + NQ * (int)ticket;
    if (t >= p.n_tasks) break;
    uint64_t ts_start = 0, ts_route = 0, ts_take = 0;
    if (p.trace) ts_start = __builtin_amdgcn_s_memrealtime();
    // The next ticket: drawn now from the queue's counter, read after this task.  Vector memory returns in issue order, so the
    // task's own loads bring the draw back with them.
    uint32_t nxt = 0, nt = 0;
    bool got = !DYN;
    // Each task reads the drawn ticket right after its loads and before its stores
    // (a read after the stores would wait for them: gfx9 counts stores in vmcnt).
    auto take = [&]() {
      if (!got) {
        nt = (uint32_t)__builtin_amdgcn_readlane((int)nxt, 0);
        got = true;
      }
      if (p.trace && !ts_take) ts_take = __builtin_amdgcn_s_memrealtime();
    };
    if (DYN && lane0 == 0) {
      // An opaque (per-lane) address keeps this one lane's atomic as it is: the
      // compiler's wave-aggregated form broadcasts the result at once, waiting for it.
      uintptr_t a = reinterpret_cast<uintptr_t>(draw);
      asm volatile("" : "+v"(a));
      nxt = __hip_atomic_fetch_add(reinterpret_cast<__attribute__((address_space(1))) uint32_t*>(a), 1u,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // The lane index is re-derived per task: otherwise every per-lane address of
    // every task type is hoisted out of this loop and held in registers throughout.
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const TaskRef tk = decode_task(p, t);
    if (!routed && (tk.type == kTG || tk.type == kTD)) {
      // The first routed task of this wave: the block's routing, resolved by this
      // wave or another of the block (one call site: the resolution is long code).
      route_fetch(p, lane, rwc, tag, err, s_rt);
      routed = true;
      if (p.trace) ts_route = __builtin_amdgcn_s_memrealtime();
    }
    if (tk.type == kTD && tk.slot == p.k - 1) {
      // The combining tasks need the weights and the gate; the first of them publishes the
      // call's routing outputs.
      if (!weighted) {
        route_weights(lane, rwc, err, s_rt);
        weighted = true;
      }
      if (tk.idx == 0) publish_routing(p, lane, rwc);
    }
    // The shared gate/up tasks (all drawn at entry) issue their loads a few us late.  Issued at
    // once, their rows sit in the memory queues in front of the router rows loaded beside them,
    // and the routing is the critical path; the shared expert has slack until the routing
    // resolves (~8 us).  Exact bf16 36.4 -> 35.3 us at the full-size layer; int4 (now that its
    // tickets are drawn too) 29.6-29.7 -> 28.4-28.5 us.
    if (tk.type == kTS && i == 0) __builtin_amdgcn_s_sleep(shared_delay<Q4>());
    if (tk.type == kTR) {
      task_router<MH, EXACT, LN>(p, tk.idx, lane, get_x, tag, take);
    } else if (tk.type == kTS || tk.type == kTG) {
      // Gate/up pairs: the shared expert (S) or routed slot j (G); one call site.
      const bool shared = tk.type == kTS;
      const int e = shared ? 0 : wave_slot_expert(p, tk.slot, rwc);
      const int n_rows = shared ? p.Is : p.I;
      if (Q4 && !shared) {
        if (e >= 0)
          up_q4<MH, kQ4Pairs, QR>(reinterpret_cast<const uint8_t*>(ld_inv(p.table + 4 * e)),
                    reinterpret_cast<const uint16_t*>(ld_inv(p.table + 4 * e + 1)), tk.idx * kQ4Pairs, p.I, p.H,
                    get_x, lane, p.act64 + (size_t)tk.slot * p.I / 2, tag, take);
      } else if (e >= 0) {
        const uint16_t* gu = shared ? nullptr : reinterpret_cast<const uint16_t*>(ld_inv(p.table + 2 * e));
        const uint16_t* g = shared ? p.sh_gate : gu;
        const uint16_t* u = shared ? p.sh_up : gu + (size_t)p.I * p.H;
        constexpr int P = Q4 ? kQ4SPairs : kPairs;
        up_pairs<MH, EXACT, P, LN && !Q4>(g, u, tk.idx * P, n_rows, p.H, get_x, lane,
                            p.act64 + (shared ? (size_t)p.k * p.I / 2 : (size_t)tk.slot * p.I / 2), tag, take);
      }
    } else if (Q4 && tk.type == kTD) {
      task_down_q4<MI, RQ, QR>(p, tk.slot, tk.idx, lane, rwc, tag, err, s_rt, take);
    } else {
      // Down rows: the shared expert (SD) or routed slot j (D); D(k-1) combines.
      const bool shared = tk.type == kTSD;
      const int e = shared ? 0 : wave_slot_expert(p, tk.slot, rwc);
      const int h0 = tk.idx * kDownRows;
      float d[kDownRows] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      uint64_t pre[kFusedMaxK];
      if (e >= 0) {
        const uint16_t* w = shared ? p.sh_down : reinterpret_cast<const uint16_t*>(ld_inv(p.table + 2 * e + 1));
        const uint64_t* a = p.act64 + (shared ? (size_t)p.k * p.I / 2 : (size_t)tk.slot * p.I / 2);
        down_dots<MI, EXACT>(w, a, p, shared ? p.Is : p.I, h0, lane, d, tag, err);
        take();
      }
      if (Q4) {
        // Int4 mode keeps one row per word: the shared rows as fp32 words of their bf16 values.
        int rows[kDownRows];
#pragma unroll
        for (int r = 0; r < kDownRows; ++r) rows[r] = __float_as_int(d[r]);
        const int row = spread(rows);
        if (lane < kDownRows) st64c(p.dq64 + (size_t)p.k * p.H + h0 + lane, tagged(tag, (uint32_t)row));
      } else if (shared || tk.slot != p.k - 1) {
        // Publish this slot's rows (a skipped slot publishes zeros the combine ignores).
        // Lane q < 4 publishes rows 2q, 2q + 1 (the row values are wave-uniform).
        int pairs[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int q2 = 0; q2 < kDownRows / 2; ++q2)
          pairs[q2] = (int)((uint32_t)f32_to_bf16(d[2 * q2]) | ((uint32_t)f32_to_bf16(d[2 * q2 + 1]) << 16));
        const int pair = spread8(pairs);
        if (lane < kDownRows / 2)
          st64c(p.dq64 + ((size_t)(shared ? p.k : tk.slot) * p.H + h0) / 2 + lane, tagged(tag, (uint32_t)pair));
      } else {
        combine_words(p, h0, lane, pre);
        combine_rows(p, e, h0, lane, d, rwc, tag, err, s_rt, pre);
      }
    }
    if (!got) {
      // A task that loaded nothing (skipped slot): the draw is read here.
      uint32_t v = nxt;
      asm volatile("" : "+v"(v));
      nt = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
    }
    if (p.trace && lane0 == 0) {
      uint64_t* rec = p.trace + kTraceHeader + (size_t)t * kTraceTaskWords;
      rec[0] = ts_start;
      rec[1] = ts_route;
      rec[2] = ts_take;
      rec[3] = __builtin_amdgcn_s_memrealtime();
      rec[4] = (uint32_t)__builtin_amdgcn_s_getreg((31 << 11) | 4);    // HW_ID
      rec[5] = (uint32_t)__builtin_amdgcn_s_getreg((31 << 11) | 20);   // XCC_ID
      rec[6] = ticket;
      rec[7] = (uint64_t)tk.type | (uint64_t)(tk.slot + 1) << 8 | (uint64_t)tk.idx << 16;
    }
    ticket = DYN ? nt : rank + users * (i + 1);
  }
  if (p.trace && lane0 == 0) {
    uint64_t* rec = p.trace + kTraceHeader + (size_t)p.n_tasks * kTraceTaskWords + 2 * ((size_t)blockIdx.x * kWaves + wid);
    rec[0] = t_entry;
    rec[1] = __builtin_amdgcn_s_memrealtime();
  }
  // The last wave to leave queue q re-zeroes its exit count; the last queue to
  // drain ends the call.
  uint32_t fin = 0;
  if (lane0 == 0) {
    if (add32c(line(p, kLnQueueExit + q), 1u) == users - 1u) {
      st32c(line(p, kLnQueueExit + q), 0u);
      st32c(draw, 0u);
      fin = add32c(line(p, kLnQueuesDone), 1u) == (uint32_t)NQ - 1u;
    }
  }
  if (__builtin_amdgcn_readfirstlane(fin)) finish_call(p, tag, lane0);
}

// ---------------------------------------------------------------- launch
typedef void (*FusedKernel)(DecodeParams);

// Exact-fit variants (H = 512 MH, I = Is = 512 MI) for the common layer widths;
// masked variants cover the rest up to H = 4096, I = Is = 2048.
// Int4 mode has exact-fit variants only.
template <bool LN>
static FusedKernel pick_fused_t(int H, int I, int Is, bool q4, bool qr) {
  if (H % 512 == 0 && I % 512 == 0 && (Is == 0 || Is == I)) {
    const int key = (H / 512) * 10 + I / 512;
    if (qr) {   // int4 with the reference's per-row fp16 scales
      switch (key) {
        case 11: return k_decode_fused<1, 1, true, true, LN, false, true>;
        case 21: return k_decode_fused<2, 1, true, true, LN, false, true>;
        case 22: return k_decode_fused<2, 2, true, true, LN, false, true>;
        case 42: return k_decode_fused<4, 2, true, true, LN, false, true>;
        case 52: return k_decode_fused<5, 2, true, true, LN, false, true>;
        case 62: return k_decode_fused<6, 2, true, true, LN, false, true>;
        case 84: return k_decode_fused<8, 4, true, true, LN, false, true>;
      }
      return nullptr;
    }
    if (q4) {
      switch (key) {
        case 11: return k_decode_fused<1, 1, true, true, LN>;
        case 21: return k_decode_fused<2, 1, true, true, LN>;
        case 22: return k_decode_fused<2, 2, true, true, LN>;
        case 42: return k_decode_fused<4, 2, true, true, LN>;
        case 52: return k_decode_fused<5, 2, true, true, LN>;
        case 62: return k_decode_fused<6, 2, true, true, LN>;
        case 84: return k_decode_fused<8, 4, true, true, LN>;
      }
      return nullptr;
    }
    switch (key) {
      case 21: return k_decode_fused<2, 1, true, false, LN>;
      case 22: return k_decode_fused<2, 2, true, false, LN>;
      case 42: return k_decode_fused<4, 2, true, false, LN>;
      case 52: return k_decode_fused<5, 2, true, false, LN>;
      case 62: return k_decode_fused<6, 2, true, false, LN>;
      case 84: return k_decode_fused<8, 4, true, false, LN>;
    }
  }
  if (q4 || qr) return nullptr;
  const int inter = I > Is ? I : Is;
  const int ncH = (H + 511) / 512, ncI = (inter + 511) / 512;
  const int mh = ncH <= 2 ? 2 : ncH <= 4 ? 4 : ncH <= 6 ? 6 : ncH <= 8 ? 8 : 0;
  const int mi = ncI <= 2 ? 2 : ncI <= 4 ? 4 : 0;
  switch (mh * 10 + mi) {
    case 22: return k_decode_fused<2, 2, false, false, LN>;
    case 24: return k_decode_fused<2, 4, false, false, LN>;
    case 42: return k_decode_fused<4, 2, false, false, LN>;
    case 44: return k_decode_fused<4, 4, false, false, LN>;
    case 62: return k_decode_fused<6, 2, false, false, LN>;
    case 64: return k_decode_fused<6, 4, false, false, LN>;
    case 82: return k_decode_fused<8, 2, false, false, LN>;
    case 84: return k_decode_fused<8, 4, false, false, LN>;
  }
  return nullptr;
}
// q4: 0 bf16 experts, 1 int4 with group-128 bf16 scales, 2 int4 with per-row fp16 scales.
static FusedKernel pick_fused(int H, int I, int Is, int q4, bool ln) {
  return ln ? pick_fused_t<true>(H, I, Is, q4 != 0, q4 == 2) : pick_fused_t<false>(H, I, Is, q4 != 0, q4 == 2);
}
// The recording twin of a block-mode exact-fit kernel, or null.
static FusedKernel pick_traced(int H, int I, int Is, int q4, bool ln) {
  if (ln || q4 == 2 || H % 512 || I % 512 || (Is != 0 && Is != I)) return nullptr;
  switch ((H / 512) * 10 + I / 512) {
    case 11: return q4 ? k_decode_fused<1, 1, true, true, false, true> : nullptr;
    case 21: return q4 ? k_decode_fused<2, 1, true, true, false, true> : k_decode_fused<2, 1, true, false, false, true>;
    case 22: return q4 ? k_decode_fused<2, 2, true, true, false, true> : k_decode_fused<2, 2, true, false, false, true>;
    case 42: return q4 ? k_decode_fused<4, 2, true, true, false, true> : k_decode_fused<4, 2, true, false, false, true>;
    case 52: return q4 ? k_decode_fused<5, 2, true, true, false, true> : k_decode_fused<5, 2, true, false, false, true>;
    case 62: return q4 ? k_decode_fused<6, 2, true, true, false, true> : k_decode_fused<6, 2, true, false, false, true>;
    case 84: return q4 ? k_decode_fused<8, 4, true, true, false, true> : k_decode_fused<8, 4, true, false, false, true>;
  }
  return nullptr;
}

// Blocks of a kernel to launch on the current device (cached): every one resident
// at once, at most kBlocksPerCU per CU.
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
  const int n = cu * (occ < 1 ? 1 : occ < kBlocksPerCU ? occ : kBlocksPerCU);
  if (used < 64) cache[used++] = {dev, k, n};
  return n;
}

// The debug timeline buffer (tmoe_debug_decode_trace): process-wide, off (null) by default.
static std::mutex g_trace_mu;
static uint64_t* g_trace = nullptr;
static size_t g_trace_bytes = 0;

int decode_fused_launch(DecodeParams& p, bool run_router, hipStream_t s) {
  const bool has_sh = p.sh_gate != nullptr;
  FusedKernel k = pick_fused(p.H, p.I, p.Is, p.q4, p.ln_w != nullptr);
  if (!k || p.k > kFusedMaxK || (has_sh && !run_router) || (p.I & 1) || (p.Is & 1) || (p.H % kDownRows))
    return TMOE_ERR_SHAPE;
  const int n_rows = (p.logits_in ? 0 : p.E) + (has_sh ? 1 : 0);
  p.n_r = run_router ? (n_rows > 0 ? (n_rows + kRouterRows - 1) / kRouterRows : 1) : 0;
  const int s_pairs = p.q4 ? kQ4SPairs : kPairs;
  p.n_s = has_sh ? (p.Is + s_pairs - 1) / s_pairs : 0;
  p.n_sd = has_sh ? p.H / kDownRows : 0;
  if (p.q4) {
    p.n_g = p.I / kQ4Pairs;
    p.n_d = p.H / q4_down_rows(p.I / 512);
  } else {
    p.n_g = (p.I + kPairs - 1) / kPairs;
    p.n_d = p.H / kDownRows;
  }
  // While the routing resolves only the router rows load: any request issued
  // behind a full memory queue waits microseconds, and every routing step is one.
  // Int4 (static tickets): S right after R.  A wave's second task is the one a grid's
  // worth of tasks after its first, so the R and S waves, done before the routing
  // resolves, take the gate/up tasks that do not fit in the first round and start them
  // with the others (S after G1 left G7 to the G0 waves, after their first task:
  // 26.7 -> 24.9 us at the full-size layer).
  p.sh_after = p.q4 ? -1 : p.k - 1 < kSharedAfter ? p.k - 1 : kSharedAfter;
  p.sd_after = p.k - 1 < p.sh_after + kDownLag ? p.k - 1 : p.sh_after + kDownLag;
  p.n_tasks = p.n_r + p.n_s + p.n_sd + p.k * (p.n_g + p.n_d);
  int grid = resident_blocks(k);
  if (grid <= 0) return TMOE_ERR_HIP;
  const int need = (p.n_tasks + kWaves - 1) / kWaves;
  if (grid > need) grid = need;
  if (grid < 32) grid = 32;   // every queue needs a wave: one block of each group
  {
    std::lock_guard<std::mutex> lock(g_trace_mu);
    p.trace = g_trace && trace_words(p.n_tasks, grid * kWaves) * 8 <= g_trace_bytes ? g_trace : nullptr;
  }
  if (p.trace) {
    FusedKernel kt = pick_traced(p.H, p.I, p.Is, p.q4, p.ln_w != nullptr);
    if (kt && resident_blocks(kt) >= grid) k = kt;
    else p.trace = nullptr;
  }
  hipLaunchKernelGGL(k, dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

}  // namespace tmoe

// Debug: every later fused-decode launch whose records fit in `bytes` writes its timeline
// into the device buffer `buf` (each launch overwrites the last); null turns it off.
extern "C" int tmoe_debug_decode_trace(void* buf, size_t bytes) {
  if (buf && ((uintptr_t)buf & 7u)) return TMOE_ERR_ALIGN;
  std::lock_guard<std::mutex> lock(tmoe::g_trace_mu);
  tmoe::g_trace = static_cast<uint64_t*>(buf);
  tmoe::g_trace_bytes = buf ? bytes : 0;
  return TMOE_OK;
}

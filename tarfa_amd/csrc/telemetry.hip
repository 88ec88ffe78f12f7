// Route telemetry on the device: the reference's per-layer route-reuse counters
// (tarfa/engine/fused_int4.py:71-95 _record_route / routing_telemetry) kept in a
// caller-owned state buffer, updated by one launch per token for every layer, so
// the decode path never synchronises the host for telemetry.
//
// Per layer, a step records the valid expert ids of that layer's call (ids in
// [0, E); the sentinel E and anything else outside is dropped, as the reference
// drops the sentinel before recording, fused_int4.py:165-169).  A step with no
// valid id records nothing (the reference returns before recording, :168).
// For a recorded step with id list C (set S) and the previous recorded sets P1
// (newest) .. P16: uses += len(C); reuse_w += |S ∩ (P1 ∪ .. ∪ Pw)| for w in 1, 2, 4,
// 8, 16; then S becomes P1.  Distinct (layer, expert) pairs ever recorded are
// counted too.
//
// State (zero-filled by the caller), per layer l:
//   u64 counters[L][8]: steps, uses, reuse_1, reuse_2, reuse_4, reuse_8, reuse_16, distinct
//   i32 history[L][16][k]: recorded sets, slot (steps % 16); -1 pads a set to k ids
//   u32 seen[L][ceil(E / 32)]: bitmap of experts ever recorded
#include "tmoe_device.h"

namespace tmoe {

constexpr int kHist = 16;
constexpr int kWindows[5] = {1, 2, 4, 8, 16};

struct TelemetryLayout {
  size_t counters, history, seen, total;
};

static TelemetryLayout telemetry_layout(int L, int k, int E) {
  TelemetryLayout t{};
  t.counters = 0;
  t.history = (size_t)L * 8 * sizeof(uint64_t);
  t.seen = t.history + (size_t)L * kHist * k * sizeof(int32_t);
  t.total = t.seen + (size_t)L * ((E + 31) / 32) * sizeof(uint32_t);
  return t;
}

// One wave per layer.  Lane j < k owns current slot j.
__global__ __launch_bounds__(64) void k_route_record(const int64_t* __restrict__ ids, int L, int k, int E,
                                                     uint64_t* __restrict__ counters, int32_t* __restrict__ history,
                                                     uint32_t* __restrict__ seen) {
  const int l = blockIdx.x;
  const int lane = threadIdx.x;
  if (l >= L) return;
  uint64_t* c = counters + (size_t)l * 8;
  int32_t* hist = history + (size_t)l * kHist * k;
  uint32_t* bits = seen + (size_t)l * ((E + 31) / 32);
  int id = -1;
  if (lane < k) {
    const int64_t e = ids[(size_t)l * k + lane];
    id = (e >= 0 && e < E) ? (int)e : -1;
  }
  // Duplicate ids within a step count once (the reference records a set).
  bool first = id >= 0;
  for (int j = 0; j < k; ++j) {
    const int other = __shfl(id, j);
    if (j < lane && other == id) first = false;
  }
  const uint64_t valid_mask = __ballot(id >= 0);   // uses count the list, duplicates included
  if (valid_mask == 0) return;                     // nothing recorded for this step
  const uint64_t steps = c[0];
  const int avail = steps < (uint64_t)kHist ? (int)steps : kHist;
  // Age of this id: 1 + how many recorded steps back it was last seen (0 = not within 16).
  int age = 0;
  if (first) {
    for (int a = 1; a <= avail && age == 0; ++a) {
      const int32_t* set = hist + (size_t)((steps - (uint64_t)a) % kHist) * k;
      for (int j = 0; j < k; ++j)
        if (set[j] == id) age = a;
    }
  }
  uint64_t add[5];
#pragma unroll
  for (int w = 0; w < 5; ++w) add[w] = (uint64_t)__popcll(__ballot(first && age > 0 && age <= kWindows[w]));
  // Distinct (layer, expert): set the bit, count the ones that were clear.
  uint32_t fresh = 0;
  if (first) {
    const uint32_t m = 1u << (id & 31);
    fresh = (atomicOr(bits + (id >> 5), m) & m) ? 0u : 1u;
  }
  const uint64_t n_fresh = (uint64_t)__popcll(__ballot(fresh != 0));
  // Every lane has read the history above before lane j < k overwrites its slot.
  __syncthreads();
  if (lane < k) {
    // The new set: valid first occurrences, padded with -1.
    hist[(size_t)(steps % kHist) * k + lane] = first ? id : -1;
  }
  if (lane == 0) {
    c[0] = steps + 1;
    c[1] += (uint64_t)__popcll(valid_mask);
#pragma unroll
    for (int w = 0; w < 5; ++w) c[2 + w] += add[w];
    c[7] += n_fresh;
  }
}

}  // namespace tmoe

using namespace tmoe;

extern "C" size_t tmoe_route_telemetry_bytes(int L, int k, int E) {
  if (L < 1 || k < 1 || k > 64 || E < 1) return 0;
  return telemetry_layout(L, k, E).total;
}

extern "C" int tmoe_route_record(const int64_t* ids, int L, int k, int E, void* state, size_t state_bytes,
                                 void* stream) {
  if (!ids || !state) return TMOE_ERR_NULL;
  if (L < 1 || k < 1 || k > 64 || E < 1) return TMOE_ERR_SHAPE;
  const TelemetryLayout t = telemetry_layout(L, k, E);
  if (state_bytes < t.total) return TMOE_ERR_WORKSPACE;
  if ((uintptr_t)state & 7u) return TMOE_ERR_ALIGN;
  char* base = (char*)state;
  hipLaunchKernelGGL(k_route_record, dim3(L), dim3(64), 0, (hipStream_t)stream, ids, L, k, E,
                     (uint64_t*)(base + t.counters), (int32_t*)(base + t.history), (uint32_t*)(base + t.seen));
  return hipGetLastError() == hipSuccess ? TMOE_OK : TMOE_ERR_HIP;
}

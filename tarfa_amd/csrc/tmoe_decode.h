// Parameter block of the batch-1 (decode) kernels, shared with the ABI layer.
#pragma once

#include <stdint.h>

namespace tmoe {

struct DecodeParams {
  const uint16_t* x;          // [H]; with ln_w: the hidden state h before the layer's RMSNorm
  const uint16_t* ln_w;       // [H] RMSNorm weight (x := bf16(rmsnorm(h) * (1 + ln_w))), or null
  float ln_eps;
  const uint16_t* resid;      // [H] residual added to the output (out = bf16(resid + y)), or null
  const uint16_t* router_w;   // [E, H] or null (logits supplied or experts-only mode)
  const float* logits_in;     // [E] or null
  const uint64_t* table;      // [E][2] gate_up / down base pointers; int4: [E][4] (packed, scales) x 2
  int q4;                     // int4 routed experts, fp32 combine: 1 group-128 bf16 scales, 2 per-row fp16 scales
  const uint16_t* sh_gate;    // [Is, H]   (null = no shared expert)
  const uint16_t* sh_up;      // [Is, H]
  const uint16_t* sh_down;    // [H, Is]
  const uint16_t* sh_gate_w;  // [H]
  const int64_t* ids_in;      // [k] experts-only mode (router skipped), else null
  const uint16_t* w_in;       // [k] bf16
  int H, E, I, k, Is;
  int n_router_blocks, n_shared_up_blocks;
  int n_up_blocks_per_expert, n_shared_down_blocks;
  uint16_t* out;              // [H]
  int64_t* ids_out;           // optional
  uint16_t* w_out;            // optional
  float* logits_out;          // optional
  uint32_t* heat;             // optional
  uint32_t* status;           // workspace status block
  uint32_t* err;              // device-detected error bits (kErrExpertId | kErrTimeout) are OR-ed here
  float* logits_ws;           // [E + 1]
  int32_t* ids_ws;            // [k]
  float* w_ws;                // [k]
  float* gs_ws;               // [1]
  uint16_t* act_ws;           // [k * I]
  uint16_t* sact_ws;          // [Is]
  uint16_t* sh_ws;            // [H]
  // fused task graph (tmoe_decode_fused)
  uint32_t* sync;             // task-graph lines
  uint64_t* lg64;             // [kLogitReplicas][lg_stride] tagged fp32 logits (index E: shared-gate logit)
  int lg_stride;              // u64 words per logit copy
  uint64_t* act64;            // [k * I / 2] tagged bf16 activation pairs, then [Is / 2] shared
  uint64_t* dq64;             // [(k + 1) * H] tagged per-slot down results (slot k: shared, before its gate):
                              // bf16 row pairs, or one fp32 row per word in int4 mode
  void* handoff;              // the fixed-size tagged hand-off area: zeroed when the epoch wraps
  size_t handoff_words;       // its size in uint64
  int n_r, n_s, n_g, n_d, n_sd, n_tasks;   // task counts: router, shared up, gate/up per slot, down per slot,
                                           // shared down; total
  int sh_after, sd_after;     // shared gate/up (S) and shared down (SD) follow these slots' gate/up tasks
  uint64_t* trace;            // debug timeline (tmoe_debug_decode_trace), or null: no records
};

// Debug timeline of one fused-decode call, in 100 MHz ticks of s_memrealtime:
// a header of kTraceHeader words (written by the first wave), then kTraceTaskWords words per
// task (start, routing known, loads returned, end, HW_ID, XCC_ID, ticket, type | (slot + 1) << 8 |
// idx << 16), then two words
// per wave (entry, exit), then eight per block (routing: poll start, logits complete, resolved,
// poll rounds, top-k selected, weights formed, 0, 0).
constexpr int kTraceHeader = 16;
constexpr int kTraceTaskWords = 8;
inline size_t trace_words(int n_tasks, int waves) {
  return (size_t)kTraceHeader + (size_t)n_tasks * kTraceTaskWords + (size_t)waves * 2 + (size_t)waves * 2;
}

}  // namespace tmoe

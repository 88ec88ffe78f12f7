// Workspace layout shared by every entry point.  One caller-owned, zero-filled
// device buffer; regions are 256-byte aligned.  Sizes are for T tokens.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace tmoe {

enum StatusSlot {
  kStatusError = 0,      // OR of device-detected error bits (kErrExpertId | kErrTimeout)
  kStatusRouterDone = 1, // arrival counter of the unfused decode router blocks
  kStatusSlots = 64,
};
enum ErrorBit { kErrExpertId = 1u, kErrTimeout = 2u };

// Synchronisation lines (the fused decode's task graph, the small-batch arrivals), at a
// fixed offset for every T so that calls of different sizes on one workspace never see
// another call's data in them.  Every counter owns a 256-byte line (64 uint32): atomics on
// one hot line serialise at ~11 ns each.  Counters are zero between calls (the last wave to
// leave a queue re-zeroes its exit count; the last small-batch block of a token or column
// tile re-zeroes its arrival count).  Hand-off words
// (logits, activations, per-slot down results) are 64-bit {payload,
// tag}: the tag is the call's epoch, so words left by earlier calls never match
// and nothing is cleared between calls.
constexpr int kLine = 64;                 // uint32 per line
// Small-batch path: 2 <= T <= kSbMaxTokens tokens, T * k <= kSbMaxEntries, at most kSbTiles
// combine tiles of 64 output columns.
constexpr int kSbMaxTokens = 16, kSbMaxEntries = 256, kSbTiles = 4096 / 64;
constexpr int kLogitReplicas = 32;        // router logits published to this many copies (blocks poll one each)
constexpr int kQueues = 128;              // task queues: 4 waves x 32 block groups (4 per XCD)
enum SyncLine {
  kLnEpoch = 0,                           // word 0: epoch of the next call (tag = epoch + 1)
  kLnQueuesDone = 1,                      // queues fully drained this call
  kLnQueue = 2,                           // [kQueues] word kQueueEpochWord: epoch copy for the queue's waves
  kLnQueueExit = kLnQueue + kQueues,      // [kQueues] waves that left each queue
  kLnSbRouter = kLnQueueExit + kQueues,   // [kSbMaxTokens] small-batch router blocks arrived, per token
  kLnSbTile = kLnSbRouter + kSbMaxTokens, // [kSbTiles] small-batch down blocks arrived, per column tile
  kSyncLines = kLnSbTile + kSbTiles,
};
// Each queue line also carries a copy of the epoch, read by that queue's waves
// (coherent loads of one line serialise, so 2048 waves must not share one word).
constexpr int kQueueEpochWord = 16;
// Each queue's exit line also holds its ticket counter (drawn once per task).
constexpr int kQueueDrawWord = 32;
// Words of a block's routing (LDS, lane layout of a wave's routing cache): the expert ids
// of slots 0..7, their bf16 weights, the shared-expert bf16 gate.
enum RouteWord { kRwId = 0, kRwW = 8, kRwGate = 16, kRouteWords = 17 };
// u64 words per logit copy: E + 1 (index E: the shared-gate logit), rounded up to whole
// 256-byte lines.
inline int logit_stride(int E) { return ((E + 1) + 31) & ~31; }

// The fused decode's tagged hand-off words live in one area of fixed size, right after the
// sync lines, sized for the largest shape any entry point accepts (E <= 1024, k <= 16,
// H, I, Is <= 4096).  Its offset depends on nothing, so no region that a T > 1 call (or
// tmoe_dispatch, which lays out with placeholder H and I) writes can overlap it: every word
// in it is zero or was written by a decode call of this workspace, under that call's tag.
constexpr int kMaxExperts = 1024, kMaxTopK = 16, kMaxDim = 4096;
constexpr size_t kHandoffWords = (size_t)kLogitReplicas * (((kMaxExperts + 1) + 31) & ~31) +
                                 ((size_t)kMaxTopK * kMaxDim + kMaxDim) / 2 + (size_t)(kMaxTopK + 1) * kMaxDim;

struct Ws {
  size_t status;   // uint32[kStatusSlots]
  size_t sync;     // uint32[kSyncLines * kLine]   fused decode task-graph lines
  size_t tagged;   // u64[kHandoffWords]   tagged logit copies [kLogitReplicas * logit_stride(E)], activation
                   // pairs [(k * I + Is) / 2], per-slot down results [(k + 1) * H] (slot k = shared expert)
  size_t logits;   // f32[T * (E + 1)]   router logits; column E = shared-gate logit (decode)
  size_t ids;      // int32[T * k]
  size_t wts;      // f32[T * k]         routing weights (bf16 values)
  size_t gs;       // f32[T]             shared-expert gate bf16(sigmoid(bf16(x . w_sg)))
  size_t act;      // bf16[(T * k + T) * max(I, Is)]   SwiGLU activations (permuted rows for T > 1)
  size_t sh;       // bf16[T * H]        shared contribution bf16(gs * shared_down)
  size_t offsets;  // int32[E + 2]       expert row offsets (+ the shared group for T > 1)
  size_t perm;     // int32[T * k]
  size_t inv;      // int32[T * k]
  size_t scratch;  // int32[E + 64]      dispatch counters
  size_t ch;       // bf16[T * k * H]    per-assignment expert outputs, unscaled (T > 1)
  size_t desc;     // int32x4[T * k / 64 + E + T / 64 + 2]   prefill M-chunk descriptors (T > 1)
  size_t xn;       // bf16[T * H]        RMSNorm of the hidden state (the layer entry points)
  size_t sbord;    // small-batch combine order: int32 rows[kSbMaxEntries], f32 weights[kSbMaxEntries],
                   // int32 counts[kSbMaxTokens]; then the down kernel's slice descriptors
                   // (16 bytes each: a header and up to kSbMaxEntries + 2 slices)
  size_t total;
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

inline Ws ws_layout(int T, int H, int E, int I, int k, int Is) {
  Ws w{};
  size_t o = 0;
  const size_t t = (size_t)(T > 0 ? T : 1);
  const size_t inter = (size_t)(I > Is ? I : Is);
  auto take = [&](size_t bytes) { const size_t at = o; o = align256(o + bytes); return at; };
  w.status = take(sizeof(uint32_t) * kStatusSlots);
  w.sync = take(sizeof(uint32_t) * kSyncLines * kLine);
  w.tagged = take(8 * kHandoffWords);
  w.logits = take(sizeof(float) * t * (size_t)(E + 1));
  w.ids = take(sizeof(int32_t) * t * (size_t)k);
  w.wts = take(sizeof(float) * t * (size_t)k);
  w.gs = take(sizeof(float) * t);
  w.act = take(2 * (t * (size_t)k + t) * inter);
  w.sh = take(2 * t * (size_t)H);
  w.offsets = take(sizeof(int32_t) * (size_t)(E + 2));
  w.perm = take(sizeof(int32_t) * t * (size_t)k);
  w.inv = take(sizeof(int32_t) * t * (size_t)k);
  w.scratch = take(sizeof(int32_t) * (size_t)(E + 64));
  w.ch = take(t > 1 ? 2 * t * (size_t)k * (size_t)H : 0);
  w.desc = take(t > 1 ? 16 * (t * (size_t)k / 64 + (size_t)E + t / 64 + 2) : 0);
  w.xn = take(2 * t * (size_t)H);
  w.sbord = take(4 * (2 * (size_t)kSbMaxEntries + kSbMaxTokens) + 16 * ((size_t)kSbMaxEntries + 3));
  w.total = o;
  return w;
}

template <typename T>
inline T* ws_ptr(void* base, size_t off) {
  return reinterpret_cast<T*>(reinterpret_cast<char*>(base) + off);
}

}  // namespace tmoe

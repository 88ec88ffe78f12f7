// Workspace layout shared by every entry point.  One caller-owned, zero-filled
// device buffer; regions are 256-byte aligned.  Sizes are for T tokens.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace tmoe {

enum StatusSlot {
  kStatusError = 0,      // OR of device-detected error bits (bit 0: expert id out of range)
  kStatusRouterDone = 1, // arrival counter of the decode router blocks
  kStatusSlots = 64,
};

struct Ws {
  size_t status;   // uint32[64]
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
  size_t ch;       // bf16[T * k * H]    weighted per-assignment expert outputs (T > 1)
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
  w.total = o;
  return w;
}

template <typename T>
inline T* ws_ptr(void* base, size_t off) {
  return reinterpret_cast<T*>(reinterpret_cast<char*>(base) + off);
}

}  // namespace tmoe

// Exact top-8 selection of up to 256 fp32 logits by one wave (decode routing).
#pragma once

#include <math.h>

#include "tmoe_device.h"

namespace tmoe {

// ---------------------------------------------------------------- top-8 selection
// Exact top-8 of up to 256 logits (4 per lane), logit descending, ties to the lower
// expert index, as one wave: each candidate becomes a 64-bit key (order-preserving
// logit bits, then the inverted index; 0 = absent, -inf or NaN, never selected), each
// lane sorts its 4 keys, then 6 bitonic merge levels over lane groups of 2 .. 64 keep
// a sorted top-8 in every lane pair (even lane: ranks 0-3, odd lane: ranks 4-7).
// Cross-lane steps are DPP moves (or one ds_bpermute at the two widest levels), so the
// dependency chain is a few dozen instructions long rather than 8 rounds of wave-wide
// max, ballot and readlane.
__device__ __forceinline__ uint64_t topk_key(float v, int e) {
  if (!(v > -INFINITY)) return 0ull;                     // -inf, NaN
  uint32_t b = __float_as_uint(v);
  if (b == 0x80000000u) b = 0u;                          // -0 ties with +0
  const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)o << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e);
}
__device__ __forceinline__ float topk_logit(uint64_t key) {
  const uint32_t o = (uint32_t)(key >> 32);
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}
__device__ __forceinline__ void ce_desc(uint64_t& a, uint64_t& b) {
  const bool sw = b > a;
  const uint64_t hi = sw ? b : a, lo = sw ? a : b;
  a = hi;
  b = lo;
}
// The key of lane (lane ^ (2^LEVEL - 1)).
template <int LEVEL>
__device__ __forceinline__ uint64_t mirror_key(uint64_t k) {
  int lo = (int)(uint32_t)k, hi = (int)(uint32_t)(k >> 32);
  if constexpr (LEVEL == 1) {
    lo = __builtin_amdgcn_mov_dpp(lo, 0xB1, 0xF, 0xF, true);      // quad_perm [1,0,3,2]
    hi = __builtin_amdgcn_mov_dpp(hi, 0xB1, 0xF, 0xF, true);
  } else if constexpr (LEVEL == 2) {
    lo = __builtin_amdgcn_mov_dpp(lo, 0x1B, 0xF, 0xF, true);      // quad_perm [3,2,1,0]
    hi = __builtin_amdgcn_mov_dpp(hi, 0x1B, 0xF, 0xF, true);
  } else if constexpr (LEVEL == 3) {
    lo = __builtin_amdgcn_mov_dpp(lo, kDppHalfMirror, 0xF, 0xF, true);
    hi = __builtin_amdgcn_mov_dpp(hi, kDppHalfMirror, 0xF, 0xF, true);
  } else if constexpr (LEVEL == 4) {
    lo = __builtin_amdgcn_mov_dpp(lo, kDppMirror, 0xF, 0xF, true);
    hi = __builtin_amdgcn_mov_dpp(hi, kDppMirror, 0xF, 0xF, true);
  } else {
    const int src = ((int)(threadIdx.x & 63) ^ ((1 << LEVEL) - 1)) * 4;
    lo = __builtin_amdgcn_ds_bpermute(src, lo);
    hi = __builtin_amdgcn_ds_bpermute(src, hi);
  }
  return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}
__device__ __forceinline__ void clean4(uint64_t (&k)[4]) {
  ce_desc(k[0], k[2]);
  ce_desc(k[1], k[3]);
  ce_desc(k[0], k[1]);
  ce_desc(k[2], k[3]);
}
template <int LEVEL>
__device__ __forceinline__ void merge_level(uint64_t (&k)[4], bool odd) {
  uint64_t c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint64_t pk = mirror_key<LEVEL>(k[3 - i]);
    // Level 1 splits the 8 keys of a lane pair (upper half to the even lane); wider
    // levels keep the upper half of the two halves' top-8s in both halves.
    c[i] = (LEVEL == 1 && odd) ? (pk < k[i] ? pk : k[i]) : (pk > k[i] ? pk : k[i]);
  }
  if constexpr (LEVEL > 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint64_t q = mirror_key<1>(c[i]);
      c[i] = odd ? (q < c[i] ? q : c[i]) : (q > c[i] ? q : c[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) k[i] = c[i];
  clean4(k);
}
// Lane r < k gets slot r's expert id (E when fewer than r + 1 candidates exist) and
// logit; every lane gets the largest logit in m (0 when none).
__device__ __forceinline__ void top8_bitonic(const float (&v)[4], int E, int k, int lane, int& my_id,
                                             float& my_lw, float& m) {
  uint64_t key[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    key[i] = e < E ? topk_key(v[i], e) : 0ull;
  }
  ce_desc(key[0], key[1]);
  ce_desc(key[2], key[3]);
  ce_desc(key[0], key[2]);
  ce_desc(key[1], key[3]);
  ce_desc(key[1], key[2]);
  const bool odd = lane & 1;
  merge_level<1>(key, odd);
  merge_level<2>(key, odd);
  merge_level<3>(key, odd);
  merge_level<4>(key, odd);
  merge_level<5>(key, odd);
  merge_level<6>(key, odd);
  // Rank r lives in lane r >> 2, register r & 3.
  const int src = (lane >> 2) & 1;
  uint64_t mine = 0ull;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int lo = __builtin_amdgcn_ds_bpermute(src * 4, (int)(uint32_t)key[j]);
    const int hi = __builtin_amdgcn_ds_bpermute(src * 4, (int)(uint32_t)(key[j] >> 32));
    if ((lane & 3) == j) mine = ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
  }
  const uint64_t top = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(key[0] >> 32), 0) << 32) |
                       (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key[0], 0);
  m = top ? topk_logit(top) : 0.f;
  if (lane < k && lane < 8 && mine) {
    my_id = (int)(0xFFFFFFFFu - (uint32_t)mine);
    my_lw = topk_logit(mine);
  }
}

}  // namespace tmoe

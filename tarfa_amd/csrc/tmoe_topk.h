// Exact top-8 selection of up to 256 fp32 logits by one wave (decode routing).
#pragma once

#include <math.h>

#include "tmoe_device.h"

namespace tmoe {

// ---------------------------------------------------------------- top-8 selection
// Exact top-8 of up to 256 logits (4 per lane), logit descending, ties to the lower
// expert index, as one wave.  A candidate's key is its order-preserving logit bits, then
// the inverted index (0 = absent, -inf or NaN: never selected).
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
// The largest u32 over the wave (every lane gets it): max within each row of 16 by DPP,
// then the four row maxima on the scalar unit.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppXor1, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppXor2, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppHalfMirror, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppMirror, 0xF, 0xF, true));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}

// Lane r < k gets slot r's expert id (E when fewer than r + 1 candidates exist) and
// logit; every lane gets the largest logit in m (0 when none).  Each lane sorts its 4
// candidates (order-preserving 32-bit logit keys, 0 = absent; equal keys keep the lower
// expert index first); a round takes the wave maximum of the lane heads on 32-bit keys, the
// unique lane holding it (or, for equal keys in several lanes, the lowest expert index among
// them) gives the slot, and that lane pops its head.  Eight short dependent rounds of
// 32-bit operations: 1.08 us for one wave on an idle MI355X, against 1.52 us for a 64-bit
// bitonic merge network over lane groups of 2 .. 64.
__device__ __forceinline__ void top8_rounds(const float (&v)[4], int E, int k, int lane, int& my_id, float& my_lw,
                                            float& m) {
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
  uint32_t kk[4], ee[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kk[i] = (uint32_t)(key[i] >> 32);
    ee[i] = 0xFFFFFFFFu - (uint32_t)key[i];
  }
  uint32_t sk[8], se[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const uint32_t mx = wave_max_u32(kk[0]);
    const uint64_t c = __ballot(kk[0] == mx);
    uint32_t win;                                       // the slot's expert (meaningful when mx != 0)
    if (__builtin_popcountll(c) == 1) {
      win = (uint32_t)__builtin_amdgcn_readlane((int)ee[0], (int)__builtin_ctzll(c));
    } else {
      // Equal keys in several lanes (or none left): the lowest expert index among them.
      uint32_t t = kk[0] == mx ? ee[0] : 0xFFFFFFFFu;
      t = min(t, (uint32_t)__builtin_amdgcn_mov_dpp((int)t, kDppXor1, 0xF, 0xF, true));
      t = min(t, (uint32_t)__builtin_amdgcn_mov_dpp((int)t, kDppXor2, 0xF, 0xF, true));
      t = min(t, (uint32_t)__builtin_amdgcn_mov_dpp((int)t, kDppHalfMirror, 0xF, 0xF, true));
      t = min(t, (uint32_t)__builtin_amdgcn_mov_dpp((int)t, kDppMirror, 0xF, 0xF, true));
      win = min(min((uint32_t)__builtin_amdgcn_readlane((int)t, 0), (uint32_t)__builtin_amdgcn_readlane((int)t, 16)),
                min((uint32_t)__builtin_amdgcn_readlane((int)t, 32), (uint32_t)__builtin_amdgcn_readlane((int)t, 48)));
    }
    sk[r] = mx;
    se[r] = win;
    if (mx != 0u && (int)(win & 63u) == lane) {
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        kk[i] = kk[i + 1];
        ee[i] = ee[i + 1];
      }
      kk[3] = 0u;
    }
  }
  uint32_t mk = 0u, me = (uint32_t)E;
#pragma unroll
  for (int r = 0; r < 8; ++r)
    if (lane == r) {
      mk = sk[r];
      me = se[r];
    }
  m = sk[0] ? topk_logit((uint64_t)sk[0] << 32) : 0.f;
  if (lane < k && lane < 8 && mk) {
    my_id = (int)me;
    my_lw = topk_logit((uint64_t)mk << 32);
  }
}

}  // namespace tmoe

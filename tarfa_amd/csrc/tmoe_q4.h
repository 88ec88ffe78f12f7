// Int4 (group-128 bf16 scale) GEMV pieces for the decode kernel.
//
// Weight row format (tarfa/engine/channel_q4.py:10-14 with a per-group scale):
// packed bytes [K/2], byte b = columns 2b (low nibble) and 2b+1 (high nibble),
// value = nibble - 8; scales [K/128] bf16.  A wave reads a row in chunks of 512
// columns: lane l takes the 4-byte word of columns c*512 + 8l .. +7 (nibble j =
// column j of the 8), the same columns as the bf16 fragment layout (XPack), so
// the 8 columns of a lane share one scale group, 4c + l/16.
//
// Dot of one word with 8 bf16 inputs, fp32 accumulation: a nibble n becomes the
// bf16 value 128 + n (bits 0x4300 | n, exact), paired columns (m, m + 4) so one
// AND-OR per pair builds it; then sum (128 + n) x - 136 sum x = sum (n - 8) x.  The
// input pairs are re-paired to (m, m + 4) once per task.  Every product is exact in
// fp32; only the accumulation rounds (the reference's Triton kernel also
// accumulates in fp32, tarfa/engine/moe_kernel.py:54-63).
#pragma once

#include "tmoe_gemv.h"

namespace tmoe {

constexpr int kQ4Group = 128;   // columns per scale group

template <int MAXC>
struct Q4Frag {
  uint32_t x[MAXC][4];   // input pairs (columns m, m + 4) of the lane's 8 columns
  float off[MAXC];       // -136 * (sum of the lane's 8 inputs)
};

template <int MAXC>
__device__ __forceinline__ void q4_prepare(const XPack<MAXC>& f, Q4Frag<MAXC>& q) {
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const u32x4 v = f.v[c];   // pairs (0,1) (2,3) (4,5) (6,7), even column in the low half
    q.x[c][0] = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);   // (0, 4)
    q.x[c][1] = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);   // (1, 5)
    q.x[c][2] = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);   // (2, 6)
    q.x[c][3] = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);   // (3, 7)
    const float s = ((bf16_lo(v.x) + bf16_hi(v.x)) + (bf16_lo(v.y) + bf16_hi(v.y))) +
                    ((bf16_lo(v.z) + bf16_hi(v.z)) + (bf16_lo(v.w) + bf16_hi(v.w)));
    q.off[c] = -136.0f * s;
  }
}

// acc + sum over the 8 columns of (128 + nibble) * x.
__device__ __forceinline__ float q4_dot8(uint32_t w, const uint32_t (&x)[4], float acc) {
  // Keeps the expansion next to its use (the scheduler would otherwise expand
  // every loaded word up front, four registers each).
  asm volatile("" : "+v"(w));
  acc = dot2bf((w & 0x000F000Fu) | 0x43004300u, x[0], acc);
  acc = dot2bf(((w >> 4) & 0x000F000Fu) | 0x43004300u, x[1], acc);
  acc = dot2bf(((w >> 8) & 0x000F000Fu) | 0x43004300u, x[2], acc);
  acc = dot2bf(((w >> 12) & 0x000F000Fu) | 0x43004300u, x[3], acc);
  return acc;
}

// Selector taking the lane's bf16 half of a scale word to an fp32 value:
// lanes with bit 4 set take the high half (odd group), the others the low half.
__device__ __forceinline__ uint32_t q4_scale_sel(int lane) { return (lane & 16) ? 0x03020C0Cu : 0x01000C0Cu; }

// The scale of this lane's group from a block of scale words held one per lane
// (`sreg` of lane i = word i): word `dw` (per lane), half chosen by `sel`.
__device__ __forceinline__ float q4_scale(uint32_t sreg, int dw, uint32_t sel) {
  const uint32_t v = (uint32_t)__builtin_amdgcn_ds_bpermute(dw * 4, (int)sreg);
  return __uint_as_float(__builtin_amdgcn_perm(0u, v, sel));
}

}  // namespace tmoe

// Per-head RMS-norm + rotary embedding of one (token, head) row, shared by the
// standalone head_norm_rope kernel and the fused Sage quantize prologue.
// Reference: src/kernels/ops.cu:87-119 (head_norm_rope_kernel), :14-29 (block_sum).
#pragma once

#include "attn_common.hpp"

namespace mxa {

enum { kRopeNone = 0, kRopeInterleaved = 1, kRopeHalf = 2 };  // reference ops.h:35

struct NormRope {
  const float* norm_w;  // [D] or null (no norm)
  float eps;
  const float* cs;      // [S, rot/2] cos (row = token), null when no rope
  const float* sn;      // [S, rot/2] sin
  int rot, mode;
};

// Element j of lane L holds channel d = (L & 31) + 32 * (2j + (L >> 5)): the
// reference's thread d sits in warp d / 32 at lane d % 32, so each 32-lane half
// of the wave reproduces one reference warp and the sum of squares below follows
// the reference's block_sum association exactly (xor butterfly 16..1 inside each
// warp, then the same butterfly over the warp partials padded with zeros).
template <int NJ>
__device__ __forceinline__ int nr_channel(int j, int lane) {
  return (lane & 31) + 32 * (2 * j + (lane >> 5));
}

__device__ __forceinline__ float xor_shfl(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// v[j]: the row's values (0 for channels >= D) on entry, the normalised, rotated
// values rounded to bf16 (returned as bits) on exit. `buf` is this wave's LDS
// scratch of at least 64 * NJ floats.
template <int NJ>
__device__ __forceinline__ void norm_rope_row(float (&v)[NJ], uint16_t (&out)[NJ], int D, int64_t s,
                                              const NormRope& nr, float* buf, int lane) {
  static_assert(NJ >= 1 && NJ <= 4, "D <= 256");
  if (nr.norm_w) {
    float part[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float x = v[j] * v[j];
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) x += xor_shfl(x, o);
      part[j] = x;  // partial of reference warp 2j + (lane >> 5)
    }
    // all warp partials in every lane: w = 2j + half
    float w8[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float mine = j < NJ ? part[j] : 0.f;
      const float other = j < NJ ? xor_shfl(part[j], 32) : 0.f;
      w8[2 * j] = lane < 32 ? mine : other;
      w8[2 * j + 1] = lane < 32 ? other : mine;
    }
    // reference second butterfly over 32 slots (slots >= 8 are zero): the offsets
    // 16 and 8 add zeros, then ((w0 + w4) + (w2 + w6)) + ((w1 + w5) + (w3 + w7))
    const float ss = ((w8[0] + w8[4]) + (w8[2] + w8[6])) + ((w8[1] + w8[5]) + (w8[3] + w8[7]));
    const float rstd = __builtin_amdgcn_rsqf(ss / float(D) + nr.eps);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int d = nr_channel<NJ>(j, lane);
      if (d < D) v[j] = v[j] * rstd * nr.norm_w[d];
    }
  }
  if (nr.mode != kRopeNone && nr.rot > 0) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) buf[nr_channel<NJ>(j, lane)] = v[j];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int half = nr.rot / 2;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int d = nr_channel<NJ>(j, lane);
      if (d < nr.rot) {
        int pair, idx;
        float other;
        if (nr.mode == kRopeInterleaved) {
          pair = d >> 1;
          idx = d & 1;
          other = buf[d ^ 1];
        } else {
          pair = d < half ? d : d - half;
          idx = d < half ? 0 : 1;
          other = buf[d < half ? d + half : d - half];
        }
        const float c = nr.cs[s * half + pair], si = nr.sn[s * half + pair];
        // (a, b) -> (a c - b s, a s + b c)
        v[j] = idx == 0 ? v[j] * c - other * si : other * si + v[j] * c;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) out[j] = f2bf(v[j]);
}

}  // namespace mxa

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

// RoPE of one pair (a, b) -> (a c - b s, a s + b c), with the roundings pinned
// (one FMA each) so every kernel that rotates produces the same bits.
__device__ __forceinline__ float rope_first(float a, float b, float c, float s) { return __builtin_fmaf(a, c, -(b * s)); }
__device__ __forceinline__ float rope_second(float a, float b, float c, float s) { return __builtin_fmaf(a, s, b * c); }

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
        v[j] = idx == 0 ? rope_first(v[j], other, c, si) : rope_second(other, v[j], c, si);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) out[j] = f2bf(v[j]);
}

// ---- D = 128 on 16 lanes ----
// One (token, head) row per 16-lane DPP row: lane i = lane & 15 holds channels
// 8i .. 8i+7 (16-byte loads), so a wave normalises four rows at once with no LDS.
// Channel d = 8i + r sits at reference thread d (warp d/32, lane d%32 = 8(i&3) + r):
// the reference's warp butterfly pairs bit 4 of d first (lane i^2), then bit 3
// (lane i^1), then bits 2, 1, 0 (inside the lane); the warp partials of the
// 128-thread block then combine as (w0 + w2) + (w1 + w3) (lanes 8 and 4 apart).
// Every addition pairs the same two values the reference adds (addition is
// commutative), so the sum of squares is bit-identical to its block_sum.
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppRowRor8 = 0x128;  // row_ror:8 (lane i <- lane (i+8) mod 16)
constexpr int kDppRowRor4 = 0x124;  // row_ror:4

__device__ __forceinline__ void load8_bf16(float (&x)[8], const uint16_t* src) {
  const u32x4 raw = *reinterpret_cast<const u32x4*>(src);
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] = bf2f(uint16_t(raw[j >> 1] >> ((j & 1) * 16)));
}
__device__ __forceinline__ u32x4 pack8_bf16(const float (&x)[8]) {
  u32x4 w;
#pragma unroll
  for (int j = 0; j < 4; ++j) w[j] = pack_bf16x2(x[2 * j], x[2 * j + 1]);
  return w;
}

// Requirements of the 16-lane form: 16-byte aligned norm weights and rope tables;
// interleaved pairs with rot % 8 == 0, half pairs with rot % 16 == 0 (the partner
// d +- rot/2 then sits in the same slot of another lane and every lane's pairs are
// whole 16-byte groups of the tables), and table offsets that fit 32 bits.
__host__ __device__ inline bool nr128_supported(const NormRope& nr, int64_t rows) {
  auto a16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  if (nr.norm_w && !a16(nr.norm_w)) return false;
  if (nr.mode == kRopeNone || nr.rot == 0) return true;
  if (nr.rot < 0 || nr.rot > 128 || !a16(nr.cs) || !a16(nr.sn) || rows * (nr.rot / 2) >= (int64_t(1) << 31))
    return false;
  return (nr.mode == kRopeInterleaved && nr.rot % 8 == 0) || (nr.mode == kRopeHalf && nr.rot % 16 == 0);
}
// Rope mode of the 16-lane form as a compile-time value.
__host__ __device__ inline int nr128_mode(const NormRope& nr) {
  return nr.mode == kRopeNone || nr.rot == 0 ? kRopeNone : nr.mode;
}

// x: this lane's 8 channels of row s (bf16 values as floats) on entry; on exit the
// normalised, rotated values rounded to bf16 (as floats). All 64 lanes must call
// it together (DPP and shuffles); `valid` false leaves x untouched (rows past S).
// MODE: the rope mode (nr128_mode); the norm is applied when nr.norm_w is set.
template <int MODE>
__device__ __forceinline__ void nr128_row(float (&x)[8], int64_t s, bool valid, const NormRope& nr, int lane) {
  const int i = lane & 15;
  const uint32_t half = uint32_t(nr.rot) / 2u;
  const uint32_t srow = valid ? uint32_t(s) * half : 0u;  // table row offset (row 0 for invalid rows)
  // tables first: their latency overlaps the reduction
  f32x4 c4[2], s4[2];
  if constexpr (MODE == kRopeInterleaved) {
    const uint32_t o = srow + (8 * i < nr.rot ? 4u * i : 0u);  // pairs 4i .. 4i+3
    c4[0] = *reinterpret_cast<const f32x4*>(nr.cs + o);
    s4[0] = *reinterpret_cast<const f32x4*>(nr.sn + o);
  } else if constexpr (MODE == kRopeHalf) {
    const int lo = 8 * i < int(half);
    const uint32_t o = srow + (8 * i < nr.rot ? (lo ? 8u * i : 8u * i - half) : 0u);  // pairs pair0 .. +7
    c4[0] = *reinterpret_cast<const f32x4*>(nr.cs + o);
    c4[1] = *reinterpret_cast<const f32x4*>(nr.cs + o + 4);
    s4[0] = *reinterpret_cast<const f32x4*>(nr.sn + o);
    s4[1] = *reinterpret_cast<const f32x4*>(nr.sn + o + 4);
  }
  if (nr.norm_w) {
    const f32x4 w0 = *reinterpret_cast<const f32x4*>(nr.norm_w + 8 * i);
    const f32x4 w1 = *reinterpret_cast<const f32x4*>(nr.norm_w + 8 * i + 4);
    float a[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) a[r] = x[r] * x[r];
#pragma unroll
    for (int r = 0; r < 8; ++r) a[r] = a[r] + dppf<kDppQuadXor2>(a[r]);  // bit 4
#pragma unroll
    for (int r = 0; r < 8; ++r) a[r] = a[r] + dppf<kDppQuadXor1>(a[r]);  // bit 3
#pragma unroll
    for (int r = 0; r < 4; ++r) a[r] = a[r] + a[r + 4];                  // bit 2
#pragma unroll
    for (int r = 0; r < 2; ++r) a[r] = a[r] + a[r + 2];                  // bit 1
    const float w = a[0] + a[1];                                          // bit 0: warp partial
    const float t = w + dppf<kDppRowRor8>(w);                             // w0 + w2, w1 + w3
    const float ss = t + dppf<kDppRowRor4>(t);                            // (w0 + w2) + (w1 + w3)
    const float rstd = __builtin_amdgcn_rsqf(ss / 128.f + nr.eps);
#pragma unroll
    for (int r = 0; r < 8; ++r) x[r] = x[r] * rstd * (r < 4 ? w0[r] : w1[r - 4]);
  }
  if constexpr (MODE == kRopeInterleaved) {
    if (8 * i < nr.rot) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float a0 = x[2 * u], b0 = x[2 * u + 1];
        x[2 * u] = rope_first(a0, b0, c4[0][u], s4[0][u]);
        x[2 * u + 1] = rope_second(a0, b0, c4[0][u], s4[0][u]);
      }
    }
  } else if constexpr (MODE == kRopeHalf) {
    // partner channel d +- half is slot r of lane i +- half/8
    const int k = int(half) / 8, lo = 8 * i < int(half);
    const int src = (lane & ~15) | ((lo ? i + k : i - k) & 15);
    float other[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) other[r] = __shfl(x[r], src, 64);
    if (8 * i < nr.rot) {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const float c = r < 4 ? c4[0][r] : c4[1][r - 4], sn = r < 4 ? s4[0][r] : s4[1][r - 4];
        x[r] = lo ? rope_first(x[r], other[r], c, sn) : rope_second(other[r], x[r], c, sn);
      }
    }
  }
  (void)valid;
#pragma unroll
  for (int r = 0; r < 8; ++r) x[r] = bf2f(f2bf(x[r]));
}

}  // namespace mxa

// Sage-style quantized attention for gfx950: INT8 Q*K^T (v_mfma_i32_32x32x32_i8)
// and OCP-e4m3 P*V (v_mfma_f32_32x32x64_f8f6f4), fp32 softmax state.
// Reference: src/kernels/attention_fp8.cu (prologue :48-127, main kernel :220-420,
// host run<D> :422-449).
//
// Workspace (all regions 256-byte aligned; see mx_sage_layout in miroxen_attn.h):
//   qi [Hq][sq_pad][D] int8    qs [Hq][sq_pad/16] f32   (Q: 16-token groups)
//   ki [Hkv][skv_pad][D] int8  ks [Hkv][skv_pad/64] f32 (K: 64-token groups, mean removed)
//   vt [Hkv][D][skv_pad] e4m3  va [Hkv][D] f32          (V^T, per-channel 448/amax)
//   km [Hkv][D] f32 (K mean)   part [2][Hkv][nb][D] f32 (kv_stats partials, nb = ceil(Skv/256))
#include <type_traits>

#include "attn_common.hpp"


namespace mxa {

namespace {

constexpr int D = 128;

// ---------------- prologue ----------------

// Per (head, 256-token block): partial K sum / Skv and partial V abs-max per
// channel (reference kv_stats_kernel, attention_fp8.cu:51-62). Partials replace
// the reference's float atomics so the K mean has one fixed summation order.
__global__ void __launch_bounds__(D) kv_stats(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                              mx_attn_params p, int nb, float* __restrict__ part) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int64_t t0 = int64_t(b) * kStatTok;
  const int64_t t1 = t0 + kStatTok < p.Skv ? t0 + kStatTok : p.Skv;
  const uint16_t* kp = k + int64_t(h) * D + d;
  const uint16_t* vp = v + int64_t(h) * D + d;
  float s = 0.f, am = 0.f;
  int64_t t = t0;
  for (; t + 8 <= t1; t += 8) {
    uint16_t kk[8], vv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      kk[j] = kp[(t + j) * p.kv_stride];
      vv[j] = vp[(t + j) * p.kv_stride];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      s += bf2f(kk[j]);
      am = fmaxf(am, fabsf(bf2f(vv[j])));
    }
  }
  for (; t < t1; ++t) {
    s += bf2f(kp[t * p.kv_stride]);
    am = fmaxf(am, fabsf(bf2f(vp[t * p.kv_stride])));
  }
  const int64_t idx = (int64_t(h) * nb + b) * D + d;
  part[idx] = s / float(p.Skv);
  part[int64_t(p.Hkv) * nb * D + idx] = am;
}

// kmean = sum of the partials in ascending block order from 0.f; vamax = max.
__global__ void __launch_bounds__(D) kv_finalize(mx_attn_params p, int nb, const float* __restrict__ part,
                                                 float* __restrict__ km, float* __restrict__ va) {
  const int h = blockIdx.x, d = threadIdx.x;
  const float* ps = part + int64_t(h) * nb * D + d;
  const float* pa = ps + int64_t(p.Hkv) * nb * D;
  float s = 0.f, am = 0.f;
  for (int b = 0; b < nb; ++b) {
    s += ps[int64_t(b) * D];
    am = fmaxf(am, pa[int64_t(b) * D]);
  }
  km[h * D + d] = s;
  va[h * D + d] = am;
}

__device__ __forceinline__ float wave_max(float x) {
  for (int off = 32; off; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
  return x;
}

// Symmetric INT8 quantization of G-token groups of one head
// (reference quant_rows_kernel, attention_fp8.cu:65-100): x' = bf16(x) - mean,
// amax over the group, inv = amax>0 ? 127/amax : 0, q = rint(x'*inv),
// scale = amax/127*mult; rows >= S are zero. 128 threads, 8 channels per load.
template <int G>
__global__ void __launch_bounds__(128) quant_rows(const uint16_t* __restrict__ x, int64_t stride, int S,
                                                  int64_t s_pad, const float* __restrict__ mean, float mult,
                                                  int8_t* __restrict__ out, float* __restrict__ scale) {
  constexpr int NV = G * D / 8 / 128;
  __shared__ float red[2];
  const int h = blockIdx.y, grp = blockIdx.x;
  float vals[NV][8], am = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = threadIdx.x + i * 128, r = vi / (D / 8), c = (vi % (D / 8)) * 8;
    const int64_t row = int64_t(grp) * G + r;
    u32x4 raw = {0, 0, 0, 0};
    if (row < S) raw = *reinterpret_cast<const u32x4*>(x + row * stride + int64_t(h) * D + c);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint16_t bits = uint16_t(raw[j >> 1] >> ((j & 1) * 16));
      float f = 0.f;
      if (row < S) {
        f = bf2f(bits);
        if (mean) f = f - mean[h * D + c + j];
      }
      vals[i][j] = f;
      am = fmaxf(am, fabsf(f));
    }
  }
  am = wave_max(am);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = am;
  __syncthreads();
  am = fmaxf(red[0], red[1]);
  const float inv = am > 0.f ? 127.f / am : 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = threadIdx.x + i * 128, r = vi / (D / 8), c = (vi % (D / 8)) * 8;
    u32x2 w = {0, 0};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int qv = int(__builtin_rintf(vals[i][j] * inv));
      w[j >> 2] |= uint32_t(qv & 0xff) << ((j & 3) * 8);
    }
    *reinterpret_cast<u32x2*>(out + (int64_t(h) * s_pad + int64_t(grp) * G + r) * D + c) = w;
  }
  if (threadIdx.x == 0) scale[int64_t(h) * (s_pad / G) + grp] = am / 127.f * mult;
}

// OCP e4m3 of two floats (round to nearest even), saturated to +/-448 first
// (v_cvt_pk_fp8_f32 itself returns NaN above 464, the reference's conversion
// saturates: __NV_SATFINITE at attention_fp8.cu:119).
__device__ __forceinline__ uint32_t e4m3x2_sat(float a, float b) {
  a = __builtin_fminf(__builtin_fmaxf(a, -448.f), 448.f);
  b = __builtin_fminf(__builtin_fmaxf(b, -448.f), 448.f);
  return uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false)) & 0xffffu;
}

// V -> e4m3 with per-channel scale 448/amax, transposed to [H][D][skv_pad]
// in natural key order (reference v_quant_kernel, attention_fp8.cu:110-127).
// One work-group per (64-key tile, head); 256 threads.
__global__ void __launch_bounds__(256) v_quant(const uint16_t* __restrict__ v, mx_attn_params p, int64_t skv_pad,
                                               const float* __restrict__ va, uint8_t* __restrict__ vt) {
  __shared__ __align__(16) uint8_t tile[D][kKvPad + 4];
  const int h = blockIdx.y, k0 = blockIdx.x * kKvPad;
  // each thread converts 8 channels of 4 keys: 64 keys x 16 chunks = 1024 chunks / 256 threads
  for (int i = threadIdx.x; i < kKvPad * (D / 8); i += 256) {
    const int key = i / (D / 8), c = (i % (D / 8)) * 8;
    const int64_t gk = k0 + key;
    u32x4 raw = {0, 0, 0, 0};
    if (gk < p.Skv) raw = *reinterpret_cast<const u32x4*>(v + gk * p.kv_stride + int64_t(h) * D + c);
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      const float a0 = va[h * D + c + j], a1 = va[h * D + c + j + 1];
      const float f0 = gk < p.Skv && a0 > 0.f ? bf2f(uint16_t(raw[j >> 1])) * (448.f / a0) : 0.f;
      const float f1 = gk < p.Skv && a1 > 0.f ? bf2f(uint16_t(raw[j >> 1] >> 16)) * (448.f / a1) : 0.f;
      const uint32_t pk = e4m3x2_sat(f0, f1);
      tile[c + j][key] = uint8_t(pk);
      tile[c + j + 1][key] = uint8_t(pk >> 8);
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < D * (kKvPad / 16); i += 256) {
    const int d = i / (kKvPad / 16), u = i % (kKvPad / 16);
    u32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = *reinterpret_cast<const uint32_t*>(&tile[d][u * 16 + 4 * j]);
    *reinterpret_cast<u32x4*>(vt + (int64_t(h) * D + d) * skv_pad + k0 + u * 16) = w;
  }
}

// ---------------- main kernel ----------------
//
// Same skeleton as the BF16 kernel: 8 waves x 32 queries (two waves per SIMD);
// the score MFMA computes S^T = K Q^T so each lane holds one query (per-lane
// softmax state); K rows are permuted so each lane's score registers are the B
// operand of the P*V MFMA directly: byte j of the 32-byte FP8 operand of wave
// half h is key 32h + j of the 64-key tile. Integer row max; sc = qs*ks folded
// into one FMA feeding v_exp_f32; P = e4m3(448 * 2^(s*sc - m - H)); l sums the
// unquantized values (reference attention_fp8.cu:306-346).
//
// Lazy max with headroom H = kSageHeadroom (log2 units): the running max m only
// moves when the tile max exceeds it by more than H, and P carries an extra
// 2^-H so it never exceeds 448. The O rescale then becomes rare; the output is
// unchanged up to rounding (softmax is invariant to the subtracted constant, and
// acc and l carry the same factor). H = 0 is the reference's exact-max rule.
//
// LDS layouts (each tile 8 KB, DMA ops of 1 KB, read addresses = one or two
// per-lane registers plus compile-time offsets, bank-conflict free):
//   K int8: [4 d-chunks of 32][64 rows][2 halves of 16 B], half XOR row bit 5;
//   V^T e4m3: [128 channel rows][64 B], 16-byte chunk XOR ((row >> 2) & 3).

constexpr int KT = 64;
constexpr int KTILEB = KT * D;        // 8 KB int8 K tile
constexpr int VTILEB = D * KT;        // 8 KB fp8 V^T tile
constexpr int STAGEB = KTILEB + VTILEB;
constexpr float kSageHeadroom = 2.f;
#ifndef MXA_SAGE_NS
#define MXA_SAGE_NS 2
#endif

// Score row m of key block kb -> key within the 64-key tile.
__device__ __forceinline__ int kperm(int kb, int m) {
  return ((m >> 2) & 1) * 32 + kb * 16 + (m >> 3) * 4 + (m & 3);
}

template <int NW>
__device__ __forceinline__ void sage_load_tile(const int8_t* ki, const uint8_t* vt, int t, unsigned char* dst,
                                               int kvh, int64_t skv_pad, int wave, int lane) {
  const int8_t* kg = ki + (int64_t(kvh) * skv_pad + int64_t(t) * KT) * D;
  const uint8_t* vg = vt + int64_t(kvh) * D * skv_pad + int64_t(t) * KT;
#pragma unroll
  for (int jj = 0; jj < 8 / NW; ++jj) {  // K: op j = d-chunk j/2, rows (j%2)*32 + lane/2
    const int j = jj * NW + wave;
    const int row = (j & 1) * 32 + (lane >> 1);
    const int h = (lane & 1) ^ ((row >> 5) & 1);
    g2lds16(kg + row * D + (j >> 1) * 32 + h * 16, (MXA_LDS void*)(dst + j * 1024));
  }
#pragma unroll
  for (int jj = 0; jj < 8 / NW; ++jj) {  // V^T: op j = channel rows j*16 + lane/4
    const int j = jj * NW + wave;
    const int row = j * 16 + (lane >> 2);
    const int lc = (lane & 3) ^ ((row >> 2) & 3);
    g2lds16(vg + int64_t(row) * skv_pad + lc * 16, (MXA_LDS void*)(dst + KTILEB + j * 1024));
  }
}

template <int NS>
__global__ void __launch_bounds__(512, 1)
sage_attn_d128(const int8_t* __restrict__ qi, const int8_t* __restrict__ ki, const uint8_t* __restrict__ vt,
               const float* __restrict__ qs, const float* __restrict__ ks, const float* __restrict__ va,
               uint16_t* __restrict__ o, mx_attn_params p, int64_t sq_pad, int64_t skv_pad) {
  constexpr int NW = 8, QT = NW * 32, OPS = 2 * (8 / NW);
  static_assert(NS >= 2 && NS <= 4, "2..4 stages");
  __shared__ __align__(16) unsigned char st0[STAGEB];
  __shared__ __align__(16) unsigned char st1[STAGEB];
  __shared__ __align__(16) unsigned char st2[STAGEB];
  __shared__ __align__(16) unsigned char st3[STAGEB];
  __shared__ uint64_t live_tiles[kMaxLiveTiles];
  auto stage = [&](auto i) __attribute__((always_inline)) -> unsigned char* {
    constexpr int I = decltype(i)::value % NS;
    if constexpr (I == 0) return st0;
    else if constexpr (I == 1) return st1;
    else if constexpr (I == 2) return st2;
    else return st3;
  };
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 31, h = lane >> 5;
  const int ntq = (p.Sq + QT - 1) / QT;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int head = L / ntq, qtile = L % ntq;
  const int kvh = head / (p.Hq / p.Hkv);
  const int q0 = qtile * QT + wave * 32;
  const int nt = (p.Skv + KT - 1) / KT;

  auto issue = [&](int t, unsigned char* dst) __attribute__((always_inline)) {
    sage_load_tile<NW>(ki, vt, t, dst, kvh, skv_pad, wave, lane);
  };
  issue(0, stage(std::integral_constant<int, 0>{}));
  if constexpr (NS > 2) if (1 < nt) issue(1, stage(std::integral_constant<int, 1>{}));
  if constexpr (NS > 3) if (2 < nt) issue(2, stage(std::integral_constant<int, 2>{}));

  // Q^T fragments: lane (n, h) holds 16 int8 channels 32c + 16h .. +15 of its query.
  const int row = q0 + n;  // < sq_pad (sq_pad is a multiple of QT)
  i32x4 qf[4];
  {
    const int8_t* src = qi + (int64_t(head) * sq_pad + row) * D + h * 16;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) qf[cc] = *reinterpret_cast<const i32x4*>(src + cc * 32);
  }
  const float qscale = qs[int64_t(head) * (sq_pad / 16) + row / 16];
  const float* kscale = ks + int64_t(kvh) * (skv_pad / KT);
  build_live<NW, KT>(live_tiles, p, nt, wave, lane);
  __syncthreads();  // bitmaps visible (once, before the pipelined loop)

  // Per-lane LDS read bases.
  const int krow = kperm(0, n);
  const int kbase = krow * 32 + ((h ^ ((krow >> 5) & 1)) << 4);
  const int vsw = (n >> 2) & 3;
  const int vbase0 = KTILEB + n * 64 + (((2 * h) ^ vsw) << 4);
  const int vbase1 = KTILEB + n * 64 + (((2 * h + 1) ^ vsw) << 4);

  f32x16 acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) acc[db] = f32x16{};
  float m = -__builtin_inff(), l = 0.f;
  constexpr int kDead = -2147483647 - 1;

  auto step = [&](int t, auto i) __attribute__((always_inline)) {
    const unsigned char* sd = stage(i);
    if (t + NS - 2 < nt) wait_vm_n<(NS - 2) * OPS>();
    else wait_vm_n<0>();
    block_sync();
    const uint64_t live = tile_live<KT>(live_tiles, p, t);
    if (t + NS - 1 < nt) issue(t + NS - 1, stage(std::integral_constant<int, decltype(i)::value + NS - 1>{}));
    const float ksc = kscale[t];

    // ---- S^T = K Q^T (int32, exact) ----
    i32x16 s[2];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const i32x4 a = *reinterpret_cast<const i32x4*>(sd + kbase + cc * 2048 + kb * 512);
        s[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, qf[cc], cc == 0 ? i32x16{} : s[kb], 0, 0, 0);
      }
    __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (j < 5) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }

    if (live != ~0ull) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int ii = 0; ii < 16; ++ii)
          if (!((live >> (h * 32 + kb * 16 + ii)) & 1)) s[kb][ii] = kDead;
    }
    int im = s[0][0];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int ii = 0; ii < 16; ++ii) im = max(im, s[kb][ii]);
    im = max(im, other_half_i(im));
    const float sc = qscale * ksc;
    const float tmax = im == kDead ? -__builtin_inff() : float(im) * sc;
    const float mnew = tmax > m + kSageHeadroom ? tmax : m;
    const float alpha = m == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(m - mnew);
    m = mnew;
    const float base = mnew == -__builtin_inff() ? 0.f : kLog2_448 - kSageHeadroom - mnew;
    float f[32];
    float ts = 0.f;
    if (live == ~0ull) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int ii = 0; ii < 16; ++ii) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(float(s[kb][ii]), sc, base));
          f[kb * 16 + ii] = e;
          ts += e;
        }
    } else {  // dead keys contribute exactly 0 (even when sc == 0)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int ii = 0; ii < 16; ++ii) {
          const int si = s[kb][ii];
          const float e = si == kDead ? 0.f : __builtin_amdgcn_exp2f(__builtin_fmaf(float(si), sc, base));
          f[kb * 16 + ii] = e;
          ts += e;
        }
    }
    ts += other_half(ts);
    l = l * alpha + ts;
    if (!__all(alpha == 1.f)) {
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[db] *= alpha;
    }
    i32x8 pf;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const uint32_t lo = uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(f[4 * w], f[4 * w + 1], 0, false));
      pf[w] = __builtin_amdgcn_cvt_pk_fp8_f32(f[4 * w + 2], f[4 * w + 3], int(lo), true);
    }

    // ---- O^T += V^T P^T (e4m3 x e4m3 -> fp32) ----
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const i32x4 a0 = *reinterpret_cast<const i32x4*>(sd + vbase0 + db * 2048);
      const i32x4 a1 = *reinterpret_cast<const i32x4*>(sd + vbase1 + db * 2048);
      const i32x8 a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
      acc[db] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, pf, acc[db], 0, 0, 0, 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (j < 2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
  };
  for (int t = 0; t < nt; t += NS) {
    step(t, std::integral_constant<int, 0>{});
    if (t + 1 < nt) step(t + 1, std::integral_constant<int, 1>{});
    if constexpr (NS > 2) if (t + 2 < nt) step(t + 2, std::integral_constant<int, 2>{});
    if constexpr (NS > 3) if (t + 3 < nt) step(t + 3, std::integral_constant<int, 3>{});
  }

  // ---- epilogue: O = acc * vamax[d] / (448 l) -> bf16 ----
  if (row < p.Sq) {
    const float* vah = va + kvh * D;
    const float inv = l > 0.f ? 1.f / (448.f * l) : 0.f;
    uint16_t* dst = o + int64_t(row) * p.o_stride + head * D + h * 4;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + g * 8 + h * 4;
        const f32x4 sv = *reinterpret_cast<const f32x4*>(vah + d);
        uint32_t* d32 = reinterpret_cast<uint32_t*>(dst + db * 32 + g * 8);
        d32[0] = pack_bf16x2(acc[db][g * 4] * sv[0] * inv, acc[db][g * 4 + 1] * sv[1] * inv);
        d32[1] = pack_bf16x2(acc[db][g * 4 + 2] * sv[2] * inv, acc[db][g * 4 + 3] * sv[3] * inv);
      }
  }
}

}  // namespace

// Workspace carve-up (kept in one place for the host code and the kernels).
mx_sage_layout sage_layout(const mx_attn_params& p) {
  mx_sage_layout L{};
  L.sq_pad = (int64_t(p.Sq) + kSqPad - 1) / kSqPad * kSqPad;
  L.skv_pad = (int64_t(p.Skv) + kKvPad - 1) / kKvPad * kKvPad;
  const int64_t nb = (int64_t(p.Skv) + kStatTok - 1) / kStatTok;
  size_t off = 0;
  auto take = [&](size_t b) {
    const size_t o = off;
    off += (b + 255) / 256 * 256;
    return o;
  };
  L.qi = take(size_t(p.Hq) * L.sq_pad * p.D);
  L.ki = take(size_t(p.Hkv) * L.skv_pad * p.D);
  L.vt = take(size_t(p.Hkv) * p.D * L.skv_pad);
  L.qs = take(sizeof(float) * p.Hq * (L.sq_pad / 16));
  L.ks = take(sizeof(float) * p.Hkv * (L.skv_pad / kKvPad));
  L.km = take(sizeof(float) * p.Hkv * p.D);
  L.va = take(sizeof(float) * p.Hkv * p.D);
  L.part = take(sizeof(float) * 2 * p.Hkv * nb * p.D);
  L.total = off;
  return L;
}

// Prologue: preconditions checked by the caller (D == 128, q/k/v 16-byte aligned,
// strides % 8 == 0, ws 256-byte aligned and large enough).
hipError_t launch_sage_quantize(const uint16_t* q, const uint16_t* k, const uint16_t* v, const mx_attn_params& p,
                                char* ws, hipStream_t s) {
  const mx_sage_layout L = sage_layout(p);
  const int nb = (p.Skv + kStatTok - 1) / kStatTok;
  float* part = reinterpret_cast<float*>(ws + L.part);
  float* km = reinterpret_cast<float*>(ws + L.km);
  float* va = reinterpret_cast<float*>(ws + L.va);
  hipLaunchKernelGGL(kv_stats, dim3(p.Hkv, nb), dim3(D), 0, s, k, v, p, nb, part);
  hipLaunchKernelGGL(kv_finalize, dim3(p.Hkv), dim3(D), 0, s, p, nb, part, km, va);
  const float qmult = p.scale * kLog2e;
  hipLaunchKernelGGL(quant_rows<16>, dim3(unsigned(L.sq_pad / 16), p.Hq), dim3(128), 0, s, q, p.q_stride, p.Sq,
                     L.sq_pad, (const float*)nullptr, qmult, reinterpret_cast<int8_t*>(ws + L.qi),
                     reinterpret_cast<float*>(ws + L.qs));
  hipLaunchKernelGGL(quant_rows<kKvPad>, dim3(unsigned(L.skv_pad / kKvPad), p.Hkv), dim3(128), 0, s, k, p.kv_stride,
                     p.Skv, L.skv_pad, (const float*)km, 1.f, reinterpret_cast<int8_t*>(ws + L.ki),
                     reinterpret_cast<float*>(ws + L.ks));
  hipLaunchKernelGGL(v_quant, dim3(unsigned(L.skv_pad / kKvPad), p.Hkv), dim3(256), 0, s, v, p, L.skv_pad,
                     (const float*)va, reinterpret_cast<uint8_t*>(ws + L.vt));
  return hipGetLastError();
}

hipError_t launch_sage_attend(uint16_t* o, const mx_attn_params& p, const char* ws, hipStream_t s) {
  constexpr int QT = 256;
  static_assert(kSqPad % QT == 0, "Q padding must cover whole query tiles");
  const mx_sage_layout L = sage_layout(p);
  const int ntq = (p.Sq + QT - 1) / QT;
  const int64_t blocks = int64_t(ntq) * p.Hq;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((sage_attn_d128<MXA_SAGE_NS>), dim3(unsigned(blocks)), dim3(512), 0, s,
                     reinterpret_cast<const int8_t*>(ws + L.qi), reinterpret_cast<const int8_t*>(ws + L.ki),
                     reinterpret_cast<const uint8_t*>(ws + L.vt), reinterpret_cast<const float*>(ws + L.qs),
                     reinterpret_cast<const float*>(ws + L.ks), reinterpret_cast<const float*>(ws + L.va), o, p,
                     L.sq_pad, L.skv_pad);
  return hipGetLastError();
}

}  // namespace mxa

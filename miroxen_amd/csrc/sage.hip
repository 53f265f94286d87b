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

#ifdef MXA_PPT
__device__ uint64_t* g_ppt = nullptr;
extern "C" int mx_debug_ppt(void* buf) {
  return hipMemcpyToSymbol(HIP_SYMBOL(g_ppt), &buf, sizeof(buf)) == hipSuccess ? 0 : -2;
}
#endif

namespace {

constexpr int D = 128;

// ---------------- prologue ----------------
//
// Three launches (the reference uses a memset and four kernels, :433-446):
//  1. prep_stats_q: blocks [0, Hkv*nb) reduce K/V statistics of one 256-token
//     block of one head; the remaining blocks quantize Q (one 16-row group per
//     wave). K/V rows are staged through LDS with 16-byte coalesced loads, then
//     each channel is summed sequentially over the block's tokens from LDS.
//  2. prep_finalize: K mean (partials summed in ascending block order from 0.f)
//     and V abs-max per (head, channel).
//  3. prep_kv_quant: per (64-key tile, head): K - mean -> INT8 with one scale per
//     tile, V -> e4m3 transposed to V^T.
// Arithmetic follows the reference's quant_rows_kernel / kv_stats_kernel /
// v_quant_kernel (attention_fp8.cu:51-127) operation for operation, so the
// quantized bytes and scales are bit-identical to the oracle's restatement.

__device__ __forceinline__ float wave_max(float x) {
  for (int off = 32; off; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
  return x;
}

// Symmetric INT8 of 8 floats with a shared inverse scale (reference :96).
__device__ __forceinline__ u32x2 quant8(const float (&x)[8], float inv) {
  u32x2 w = {0, 0};
#pragma unroll
  for (int j = 0; j < 8; ++j) w[j >> 2] |= uint32_t(int(__builtin_rintf(x[j] * inv)) & 0xff) << ((j & 3) * 8);
  return w;
}

constexpr int kStatChunk = 128;  // tokens staged in LDS per step of a stats block

__global__ void __launch_bounds__(256) prep_stats_q(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                    const uint16_t* __restrict__ v, mx_attn_params p, int nb,
                                                    float qmult, int64_t sq_pad, float* __restrict__ part,
                                                    int8_t* __restrict__ qi, float* __restrict__ qs) {
  __shared__ __align__(16) uint16_t kt[kStatChunk * D];
  __shared__ __align__(16) uint16_t vt_[kStatChunk * D];
  const int tid = threadIdx.x, nstat = p.Hkv * nb;
  if (int(blockIdx.x) < nstat) {
    // ---- K sum / V abs-max over tokens [b*256, min(b*256+256, Skv)) of head h ----
    const int h = blockIdx.x / nb, b = blockIdx.x % nb;
    const int64_t t0 = int64_t(b) * kStatTok;
    const int64_t t1 = t0 + kStatTok < p.Skv ? t0 + kStatTok : p.Skv;
    float sum = 0.f, am = 0.f;
    for (int64_t c0 = t0; c0 < t1; c0 += kStatChunk) {
      const int rows = int(t1 - c0 < kStatChunk ? t1 - c0 : kStatChunk);
      for (int i = tid; i < rows * (D / 8); i += 256) {
        const int r = i / (D / 8), c = (i % (D / 8)) * 8;
        const int64_t g = (c0 + r) * p.kv_stride + int64_t(h) * D + c;
        *reinterpret_cast<u32x4*>(&kt[r * D + c]) = *reinterpret_cast<const u32x4*>(k + g);
        *reinterpret_cast<u32x4*>(&vt_[r * D + c]) = *reinterpret_cast<const u32x4*>(v + g);
      }
      __syncthreads();
      if (tid < D) {
#pragma unroll 16
        for (int r = 0; r < rows; ++r) sum += bf2f(kt[r * D + tid]);  // sequential, token order
      } else {
        const int d = tid - D;
#pragma unroll 16
        for (int r = 0; r < rows; ++r) am = fmaxf(am, fabsf(bf2f(vt_[r * D + d])));
      }
      __syncthreads();
    }
    if (tid < D) part[(int64_t(h) * nb + b) * D + tid] = sum / float(p.Skv);
    else part[int64_t(p.Hkv) * nb * D + (int64_t(h) * nb + b) * D + (tid - D)] = am;
    return;
  }
  // ---- Q: one 16-row group per wave; lane owns 4 chunks of 8 channels ----
  const int wave = tid >> 6, lane = tid & 63;
  const int64_t gid = (int64_t(blockIdx.x) - nstat) * 4 + wave;  // group index over (head, group)
  const int ng = int(sq_pad / 16);
  if (gid >= int64_t(p.Hq) * ng) return;
  const int h = int(gid / ng), grp = int(gid % ng);
  float x[4][8], am = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ci = lane + i * 64, r = ci >> 4, c = (ci & 15) * 8;
    const int64_t row = int64_t(grp) * 16 + r;
    u32x4 raw = {0, 0, 0, 0};
    if (row < p.Sq) raw = *reinterpret_cast<const u32x4*>(q + row * p.q_stride + int64_t(h) * D + c);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x[i][j] = bf2f(uint16_t(raw[j >> 1] >> ((j & 1) * 16)));
      am = fmaxf(am, fabsf(x[i][j]));
    }
  }
  am = wave_max(am);
  const float inv = am > 0.f ? 127.f / am : 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ci = lane + i * 64, r = ci >> 4, c = (ci & 15) * 8;
    *reinterpret_cast<u32x2*>(qi + (int64_t(h) * sq_pad + int64_t(grp) * 16 + r) * D + c) = quant8(x[i], inv);
  }
  if (lane == 0) qs[int64_t(h) * (sq_pad / 16) + grp] = am / 127.f * qmult;
}

// kmean = sum of the partials in ascending block order from 0.f; vamax = max.
__global__ void __launch_bounds__(D) prep_finalize(mx_attn_params p, int nb, const float* __restrict__ part,
                                                   float* __restrict__ km, float* __restrict__ va) {
  const int h = blockIdx.x, d = threadIdx.x;
  const float* ps = part + int64_t(h) * nb * D + d;
  const float* pa = ps + int64_t(p.Hkv) * nb * D;
  float s = 0.f, am = 0.f;
  constexpr int B = 16;
  for (int b0 = 0; b0 < nb; b0 += B) {
    float xs[B], xa[B];
#pragma unroll
    for (int j = 0; j < B; ++j) {  // issue the batch's loads before summing
      xs[j] = b0 + j < nb ? ps[int64_t(b0 + j) * D] : 0.f;
      xa[j] = b0 + j < nb ? pa[int64_t(b0 + j) * D] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < B; ++j)
      if (b0 + j < nb) {
        s += xs[j];
        am = fmaxf(am, xa[j]);
      }
  }
  km[h * D + d] = s;
  va[h * D + d] = am;
}

// OCP e4m3 of two floats (round to nearest even), saturated to +/-448 first
// (v_cvt_pk_fp8_f32 itself returns NaN above 464; the reference's conversion
// saturates: __NV_SATFINITE at attention_fp8.cu:119).
__device__ __forceinline__ uint32_t e4m3x2_sat(float a, float b) {
  a = __builtin_fminf(__builtin_fmaxf(a, -448.f), 448.f);
  b = __builtin_fminf(__builtin_fmaxf(b, -448.f), 448.f);
  return uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false)) & 0xffffu;
}

// Per (64-key tile, head): K - mean -> INT8 (one scale per tile) and V -> e4m3
// transposed to [H][D][skv_pad] in natural key order. Thread tid owns channel
// chunk tid%16 (8 channels) of rows tid/16 + 16*i, i = 0..3.
__global__ void __launch_bounds__(256) prep_kv_quant(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                     mx_attn_params p, int64_t skv_pad,
                                                     const float* __restrict__ km, const float* __restrict__ va,
                                                     int8_t* __restrict__ ki, float* __restrict__ ks,
                                                     uint8_t* __restrict__ vt) {
  __shared__ __align__(16) uint8_t tile[D][kKvPad + 16];
  __shared__ float red[4];
  const int h = blockIdx.y, k0 = blockIdx.x * kKvPad, tid = threadIdx.x;
  const int c = (tid & 15) * 8, r0 = tid >> 4;
  float mean[8], vsc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    mean[j] = km[h * D + c + j];
    const float a = va[h * D + c + j];
    vsc[j] = a > 0.f ? 448.f / a : 0.f;
  }
  u32x4 kraw[4], vraw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = k0 + r0 + 16 * i;
    kraw[i] = vraw[i] = u32x4{0, 0, 0, 0};
    if (row < p.Skv) {
      const int64_t g = row * p.kv_stride + int64_t(h) * D + c;
      kraw[i] = *reinterpret_cast<const u32x4*>(k + g);
      vraw[i] = *reinterpret_cast<const u32x4*>(v + g);
    }
  }
  // K: x' = bf16(x) - mean (rows >= Skv are 0), amax over the tile
  float x[4][8], am = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool ok = k0 + r0 + 16 * i < p.Skv;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x[i][j] = ok ? bf2f(uint16_t(kraw[i][j >> 1] >> ((j & 1) * 16))) - mean[j] : 0.f;
      am = fmaxf(am, fabsf(x[i][j]));
    }
  }
  // V -> e4m3 into the transposed LDS tile while the K amax reduces
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = r0 + 16 * i;
    const bool ok = k0 + key < p.Skv;
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      const float f0 = ok && vsc[j] > 0.f ? bf2f(uint16_t(vraw[i][j >> 1])) * vsc[j] : 0.f;
      const float f1 = ok && vsc[j + 1] > 0.f ? bf2f(uint16_t(vraw[i][j >> 1] >> 16)) * vsc[j + 1] : 0.f;
      const uint32_t pk = e4m3x2_sat(f0, f1);
      tile[c + j][key] = uint8_t(pk);
      tile[c + j + 1][key] = uint8_t(pk >> 8);
    }
  }
  am = wave_max(am);
  if ((tid & 63) == 0) red[tid >> 6] = am;
  __syncthreads();
  am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float inv = am > 0.f ? 127.f / am : 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    *reinterpret_cast<u32x2*>(ki + (int64_t(h) * skv_pad + k0 + r0 + 16 * i) * D + c) = quant8(x[i], inv);
  if (tid == 0) ks[int64_t(h) * (skv_pad / kKvPad) + blockIdx.x] = am / 127.f * 1.f;
  // V^T rows: channel d, 64 keys = 4 x 16 bytes
  for (int i = tid; i < D * (kKvPad / 16); i += 256) {
    const int d = i / (kKvPad / 16), u = i % (kKvPad / 16);
    *reinterpret_cast<u32x4*>(vt + (int64_t(h) * D + d) * skv_pad + k0 + u * 16) =
        *reinterpret_cast<const u32x4*>(&tile[d][u * 16]);
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
// Tiles arrive by buffer_load ... lds (no VGPR staging), one K and one V^T op per
// wave per tile, placed between the score MFMAs of the previous tile.
//
// Two work-group schedules (MXA_SAGE_KIND): 8 (default) lockstep, every wave
// runs S -> softmax -> P*V per tile; 9 ping-pong, as the BF16 kernel's default.
// The softmax here is the larger share of the work (the INT8/FP8 MFMAs take half
// the cycles of BF16 ones), and a single wave alone on a SIMD runs it slower than
// two interleaved waves, so lockstep measures ~10% faster.

constexpr int KT = 64;
constexpr int KTILEB = KT * D;        // 8 KB int8 K tile
constexpr int VTILEB = D * KT;        // 8 KB fp8 V^T tile
constexpr int STAGEB = KTILEB + VTILEB;
constexpr float kSageHeadroom = 2.f;
constexpr int kScoreBias = 0x4B400000;  // bits of 12582912.0f = 1.5 * 2^23
constexpr i32x16 kScoreBias16 = {kScoreBias, kScoreBias, kScoreBias, kScoreBias, kScoreBias, kScoreBias,
                                 kScoreBias, kScoreBias, kScoreBias, kScoreBias, kScoreBias, kScoreBias,
                                 kScoreBias, kScoreBias, kScoreBias, kScoreBias};
#ifndef MXA_SAGE_NS
#define MXA_SAGE_NS 2
#endif
#ifndef MXA_SAGE_KIND
#define MXA_SAGE_KIND 8
#endif

// Score row m of key block kb -> key within the 64-key tile.
__device__ __forceinline__ int kperm(int kb, int m) {
  return ((m >> 2) & 1) * 32 + kb * 16 + (m >> 3) * 4 + (m & 3);
}

// DMA of one tile (K 8 KB + V^T 8 KB, 8 ops of 1 KB each) by NW waves; op j:
// K rows (j&1)*32 + lane/2 of d-chunk j/2 (16-byte half XOR row bit 5), V^T
// channel rows j*16 + lane/4 (16-byte chunk XOR ((row >> 2) & 3)); wave w issues
// ops j = jj*NW + w. Per-head buffer resources; the per-lane part of each address
// is loop-invariant (NW even, so j&1 == w&1), the tile and op parts are scalar.
struct SageAddr {
  __amdgpu_buffer_rsrc_t rk, rv;
  uint32_t lk, lv;  // per-lane byte offsets
};
__device__ __forceinline__ SageAddr sage_addr(const int8_t* ki, const uint8_t* vt, int kvh, int64_t skv_pad, int wave,
                                              int lane) {
  SageAddr a;
  a.rk = buf_rsrc(ki + int64_t(kvh) * skv_pad * D, uint32_t(skv_pad * D));
  a.rv = buf_rsrc(vt + int64_t(kvh) * D * skv_pad, uint32_t(skv_pad * D));
  const int krow = (wave & 1) * 32 + (lane >> 1);
  a.lk = uint32_t(krow * D + (((lane & 1) ^ ((krow >> 5) & 1)) << 4));
  const int vrow = lane >> 2;  // + j*16: scalar part (does not change the XOR term)
  a.lv = uint32_t(vrow) * uint32_t(skv_pad) + uint32_t(((lane & 3) ^ ((vrow >> 2) & 3)) << 4);
  return a;
}
// K tile tk into kdst and V^T tile tv into vdst.
template <int NW>
__device__ __forceinline__ void sage_load_tile(const SageAddr& a, int tk, int tv, unsigned char* kdst,
                                               unsigned char* vdst, int wave, int64_t skv_pad) {
  static_for<8 / NW>([&](auto jjc) __attribute__((always_inline)) {
    const int j = decltype(jjc)::value * NW + wave;
    buf2lds16(a.rk, a.lk, uint32_t((j >> 1) * 32 + tk * (KT * D)), (MXA_LDS void*)(kdst + j * 1024));
    buf2lds16(a.rv, a.lv, uint32_t(j * 16) * uint32_t(skv_pad) + uint32_t(tv * KT), (MXA_LDS void*)(vdst + j * 1024));
  });
}
// K tile tk only.
template <int NW>
__device__ __forceinline__ void sage_load_k(const SageAddr& a, int tk, unsigned char* kdst, int wave) {
  static_for<8 / NW>([&](auto jjc) __attribute__((always_inline)) {
    const int j = decltype(jjc)::value * NW + wave;
    buf2lds16(a.rk, a.lk, uint32_t((j >> 1) * 32 + tk * (KT * D)), (MXA_LDS void*)(kdst + j * 1024));
  });
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

  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const SageAddr sa = sage_addr(ki, vt, kvh, skv_pad, wave_u, lane);
  auto issue = [&](int t, unsigned char* dst) __attribute__((always_inline)) {
    sage_load_tile<NW>(sa, t, t, dst, dst + KTILEB, wave_u, skv_pad);
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
  // Dead keys get the bits of -inf: below every biased score as an integer (so the
  // integer max skips them) and, as a float, exp2(fma(-inf, sc, nm)) = 0 exactly
  // for sc > 0 (sc is clamped to >= 1e-30, which moves no live exponent).
  constexpr int kDead = int(0xFF800000u);

  auto step = [&](int t, auto i) __attribute__((always_inline)) {
    const unsigned char* sd = stage(i);
    if (t + NS - 2 < nt) wait_vm_n<(NS - 2) * OPS>();
    else wait_vm_n<0>();
    block_sync();
    const uint64_t live = tile_live<KT>(live_tiles, p, t);
    // tile index clamped: the two DMA ops are unconditional and interleave with the MFMAs
    issue(t + NS - 1 < nt ? t + NS - 1 : nt - 1, stage(std::integral_constant<int, decltype(i)::value + NS - 1>{}));
    const float ksc = kscale[t];

    // ---- S^T = K Q^T (int32, exact) ----
    i32x16 s[2];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const i32x4 a = *reinterpret_cast<const i32x4*>(sd + kbase + cc * 2048 + kb * 512);
        // accumulate on top of the bias 0x4B400000: the float with those bits + s is
        // exactly 12582912 + s (|s| < 2^22), so no int->float conversion is needed
        s[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, qf[cc], cc == 0 ? kScoreBias16 : s[kb], 0, 0, 0);
      }
    __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (j == 1 || j == 4) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      if (j < 5) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }

    if (live != ~0ull) {
      // this lane's 32 keys are bits 32h .. 32h+31: select the word once, then
      // every test is a compile-time bit position (no per-lane mask registers)
      const uint32_t lw = h ? uint32_t(live >> 32) : uint32_t(live);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int ii = 0; ii < 16; ++ii)
          if (!((lw >> (kb * 16 + ii)) & 1u)) s[kb][ii] = kDead;
    }
    int im = s[0][0];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int ii = 0; ii < 16; ++ii) im = max(im, s[kb][ii]);
    im = max(im, other_half_i(im));
    const float sc = fmaxf(qscale * ksc, 1e-30f);
    const float tmax = im == kDead ? -__builtin_inff() : float(im - kScoreBias) * sc;
    const float mnew = tmax > m + kSageHeadroom ? tmax : m;
    const float alpha = m == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(m - mnew);
    m = mnew;
    // exponent = (12582912 + s)*sc + nm with nm = (log2 448 - H - m) - 12582912*sc
    // (reference attention_fp8.cu:331, :337, plus the headroom H)
    const float nm =
        mnew == -__builtin_inff() ? -__builtin_inff() : (kLog2_448 - kSageHeadroom - mnew) - 12582912.f * sc;
    // P = 2^exponent packed to e4m3 four at a time: byte j of the 32-byte B operand
    // is key 32h + j (j = kb*16 + ii); l sums the unquantized values
    float ts = 0.f;
    i32x8 pf;
    auto pexp = [&](int si, auto masked) __attribute__((always_inline)) -> float {
      const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(__int_as_float(si), sc, nm));
      if constexpr (decltype(masked)::value) return si == kDead ? 0.f : e;
      return e;
    };
    auto pack = [&](auto masked) __attribute__((always_inline)) {
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        const int kb = w >> 2, i0 = (w & 3) * 4;
        const float e0 = pexp(s[kb][i0], masked), e1 = pexp(s[kb][i0 + 1], masked);
        const float e2 = pexp(s[kb][i0 + 2], masked), e3 = pexp(s[kb][i0 + 3], masked);
        ts += (e0 + e1) + (e2 + e3);
        const uint32_t lo = uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(e0, e1, 0, false));
        pf[w] = __builtin_amdgcn_cvt_pk_fp8_f32(e2, e3, int(lo), true);
      }
    };
    pack(std::false_type{});
    ts += other_half(ts);
    l = l * alpha + ts;
    if (!__all(alpha == 1.f)) {
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[db] *= alpha;
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

  wait_vm_n<0>();  // no LDS-DMA may land after the work-group ends
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

// ---------------- ping-pong variant ----------------
// Same data flow, but waves w and w + 4 (one SIMD) run the per-tile program one
// period apart: in each period one issues the MFMAs (P V(t), S(t+1)) while the
// other runs the softmax, separated by two work-group barriers per tile:
//   period 2t+1: A: P V(t), S(t+1)    B: softmax(t)
//   period 2t+2: A: softmax(t+1)       B: P V(t), S(t+1)
// Group A issues the DMA of K(t+2) and V(t+1) (into the buffers of K(t) and
// V(t-1), last read in period 2t) between its MFMAs in period 2t+1.
__global__ void __launch_bounds__(512, 1)
sage_attn_d128_pp(const int8_t* __restrict__ qi, const int8_t* __restrict__ ki, const uint8_t* __restrict__ vt,
                  const float* __restrict__ qs, const float* __restrict__ ks, const float* __restrict__ va,
                  uint16_t* __restrict__ o, mx_attn_params p, int64_t sq_pad, int64_t skv_pad) {
  constexpr int NW = 8, QT = NW * 32;
  __shared__ __align__(16) unsigned char kb0[KTILEB];
  __shared__ __align__(16) unsigned char kb1[KTILEB];
  __shared__ __align__(16) unsigned char vb0[VTILEB];
  __shared__ __align__(16) unsigned char vb1[VTILEB];
  __shared__ uint64_t live_tiles[kMaxLiveTiles];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 31, h = lane >> 5;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const bool group_a = wave < 4;
  const int ntq = (p.Sq + QT - 1) / QT;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int head = L / ntq, qtile = L % ntq;
  const int kvh = head / (p.Hq / p.Hkv);
  const int q0 = qtile * QT + wave * 32;
  const int nt = (p.Skv + KT - 1) / KT;
  const SageAddr sa8 = sage_addr(ki, vt, kvh, skv_pad, wave_u, lane);
  const SageAddr sa4 = sage_addr(ki, vt, kvh, skv_pad, wave_u & 3, lane);
  sage_load_tile<8>(sa8, 0, 0, kb0, vb0, wave_u, skv_pad);
  if (nt > 1) sage_load_k<8>(sa8, 1, kb1, wave_u);

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

  const int krow = kperm(0, n);
  const int kbase = krow * 32 + ((h ^ ((krow >> 5) & 1)) << 4);
  const int vsw = (n >> 2) & 3;
  const int vbase0 = n * 64 + (((2 * h) ^ vsw) << 4);
  const int vbase1 = n * 64 + (((2 * h + 1) ^ vsw) << 4);

  f32x16 acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) acc[db] = f32x16{};
  float m = -__builtin_inff(), l = 0.f;
  // Dead keys get the bits of -inf: below every biased score as an integer (so the
  // integer max skips them) and, as a float, exp2(fma(-inf, sc, nm)) = 0 exactly
  // for sc > 0 (sc is clamped to >= 1e-30, which moves no live exponent).
  constexpr int kDead = int(0xFF800000u);
  i32x16 s[2];  // biased int32 scores of the pending tile
  i32x8 pf;     // P of the pending tile (e4m3)

  auto scores = [&](const unsigned char* kd, auto ld) __attribute__((always_inline)) {
#pragma unroll
    for (int cc = 0; cc < 4; ++cc)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const i32x4 a = *reinterpret_cast<const i32x4*>(kd + kbase + cc * 2048 + kb * 512);
        s[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, qf[cc], cc == 0 ? kScoreBias16 : s[kb], 0, 0, 0);
      }
    __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (decltype(ld)::value && (j == 1 || j == 5)) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      if (j < 5) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  };
  auto pv = [&](const unsigned char* vd, auto ld) __attribute__((always_inline)) {
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const i32x4 a0 = *reinterpret_cast<const i32x4*>(vd + vbase0 + db * 2048);
      const i32x4 a1 = *reinterpret_cast<const i32x4*>(vd + vbase1 + db * 2048);
      const i32x8 a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
      acc[db] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, pf, acc[db], 0, 0, 0, 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (decltype(ld)::value) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      if (j < 2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
  };
  auto softmax = [&](int t) __attribute__((always_inline)) {
    const uint64_t live = tile_live<KT>(live_tiles, p, t);
    if (live != ~0ull) {
      // this lane's 32 keys are bits 32h .. 32h+31: select the word once, then
      // every test is a compile-time bit position (no per-lane mask registers)
      const uint32_t lw = h ? uint32_t(live >> 32) : uint32_t(live);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int ii = 0; ii < 16; ++ii)
          if (!((lw >> (kb * 16 + ii)) & 1u)) s[kb][ii] = kDead;
    }
    int im = s[0][0];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int ii = 0; ii < 16; ++ii) im = max(im, s[kb][ii]);
    im = max(im, other_half_i(im));
    const float sc = fmaxf(qscale * kscale[t], 1e-30f);
    const float tmax = im == kDead ? -__builtin_inff() : float(im - kScoreBias) * sc;
    const float mnew = tmax > m + kSageHeadroom ? tmax : m;
    const float alpha = m == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(m - mnew);
    m = mnew;
    const float nm =
        mnew == -__builtin_inff() ? -__builtin_inff() : (kLog2_448 - kSageHeadroom - mnew) - 12582912.f * sc;
    float ts = 0.f;
    auto pexp = [&](int si, auto masked) __attribute__((always_inline)) -> float {
      const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(__int_as_float(si), sc, nm));
      if constexpr (decltype(masked)::value) return si == kDead ? 0.f : e;
      return e;
    };
    auto pack = [&](auto masked) __attribute__((always_inline)) {
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        const int kb = w >> 2, i0 = (w & 3) * 4;
        const float e0 = pexp(s[kb][i0], masked), e1 = pexp(s[kb][i0 + 1], masked);
        const float e2 = pexp(s[kb][i0 + 2], masked), e3 = pexp(s[kb][i0 + 3], masked);
        ts += (e0 + e1) + (e2 + e3);
        const uint32_t lo = uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(e0, e1, 0, false));
        pf[w] = __builtin_amdgcn_cvt_pk_fp8_f32(e2, e3, int(lo), true);
      }
    };
    pack(std::false_type{});
    ts += other_half(ts);
    l = l * alpha + ts;
    if (!__all(alpha == 1.f)) {
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[db] *= alpha;
    }
  };
  // MFMA period of tile t (S(t+1) on a stale buffer when t + 1 == nt is never read).
  auto mfma_part = [&](int t, const unsigned char* kc1, const unsigned char* vcur, unsigned char* kfree,
                       unsigned char* vfree, auto ld) __attribute__((always_inline)) {
    __builtin_amdgcn_s_setprio(1);
    if constexpr (decltype(ld)::value)  // K(t+2), V(t+1), clamped so the ops are unconditional
      sage_load_tile<4>(sa4, t + 2 < nt ? t + 2 : nt - 1, t + 1 < nt ? t + 1 : nt - 1, kfree, vfree, wave_u & 3,
                        skv_pad);
    pv(vcur, ld);
    scores(kc1, ld);
    __builtin_amdgcn_s_setprio(0);
  };

  wait_vm_n<0>();
  __syncthreads();  // K(0), V(0), K(1) and the liveness bitmaps are visible
  if (group_a) scores(kb0, std::false_type{});  // period -1: S_A(0)
  block_sync();
  if (group_a) softmax(0);  // period 0: A softmax(0), B S_B(0)
  else scores(kb0, std::false_type{});

  // Tile t: kc1 = K(t+1), vcur = V(t); kfree / vfree receive K(t+2) / V(t+1).
#ifdef MXA_PPT
  uint64_t pt0 = 0, pt1 = 0, pt2 = 0, pt3 = 0, pt4 = 0;
#define MXA_PT(v) do { if (t == 20) { __builtin_amdgcn_sched_barrier(0); v = __builtin_amdgcn_s_memtime(); __builtin_amdgcn_sched_barrier(0); } } while (0)
#else
#define MXA_PT(v) do { } while (0)
#endif
  auto tile = [&](int t, const unsigned char* kc1, const unsigned char* vcur, unsigned char* kfree,
                  unsigned char* vfree) __attribute__((always_inline)) {
    MXA_PT(pt0);
    wait_vm_n<0>();  // group A: its DMA of K(t+1), V(t) landed
    block_sync();
    MXA_PT(pt1);
    if (group_a) mfma_part(t, kc1, vcur, kfree, vfree, std::true_type{});
    else softmax(t);
    MXA_PT(pt2);
    block_sync();
    MXA_PT(pt3);
    if (group_a) {
      if (t + 1 < nt) softmax(t + 1);
    } else {
      mfma_part(t, kc1, vcur, kfree, vfree, std::false_type{});
    }
    MXA_PT(pt4);
  };
  for (int t = 0; t < nt; t += 2) {
    tile(t, kb1, vb0, kb0, vb1);
    if (t + 1 < nt) tile(t + 1, kb0, vb1, kb1, vb0);
  }
  wait_vm_n<0>();  // no LDS-DMA may land after the work-group ends
#ifdef MXA_PPT
  if (lane == 0 && g_ppt) {
    uint64_t* d = g_ppt + (int64_t(blockIdx.x) * 8 + wave) * 5;
    d[0] = pt0; d[1] = pt1; d[2] = pt2; d[3] = pt3; d[4] = pt4;
  }
#endif
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
  const int64_t qgroups = int64_t(p.Hq) * (L.sq_pad / 16);
  const int64_t blocks1 = int64_t(p.Hkv) * nb + (qgroups + 3) / 4;
  if (blocks1 > 0x7fffffff) return hipErrorInvalidValue;
  const float qmult = p.scale * kLog2e;
  hipLaunchKernelGGL(prep_stats_q, dim3(unsigned(blocks1)), dim3(256), 0, s, q, k, v, p, nb, qmult, L.sq_pad, part,
                     reinterpret_cast<int8_t*>(ws + L.qi), reinterpret_cast<float*>(ws + L.qs));
  hipLaunchKernelGGL(prep_finalize, dim3(p.Hkv), dim3(D), 0, s, p, nb, (const float*)part, km, va);
  hipLaunchKernelGGL(prep_kv_quant, dim3(unsigned(L.skv_pad / kKvPad), p.Hkv), dim3(256), 0, s, k, v, p, L.skv_pad,
                     (const float*)km, (const float*)va, reinterpret_cast<int8_t*>(ws + L.ki),
                     reinterpret_cast<float*>(ws + L.ks), reinterpret_cast<uint8_t*>(ws + L.vt));
  return hipGetLastError();
}

hipError_t launch_sage_attend(uint16_t* o, const mx_attn_params& p, const char* ws, hipStream_t s) {
  constexpr int QT = 256;
  static_assert(kSqPad % QT == 0, "Q padding must cover whole query tiles");
  const mx_sage_layout L = sage_layout(p);
  const int ntq = (p.Sq + QT - 1) / QT;
  const int64_t blocks = int64_t(ntq) * p.Hq;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
#if MXA_SAGE_KIND == 9
  hipLaunchKernelGGL(sage_attn_d128_pp, dim3(unsigned(blocks)), dim3(512), 0, s,
#else
  hipLaunchKernelGGL((sage_attn_d128<MXA_SAGE_NS>), dim3(unsigned(blocks)), dim3(512), 0, s,
#endif
                     reinterpret_cast<const int8_t*>(ws + L.qi), reinterpret_cast<const int8_t*>(ws + L.ki),
                     reinterpret_cast<const uint8_t*>(ws + L.vt), reinterpret_cast<const float*>(ws + L.qs),
                     reinterpret_cast<const float*>(ws + L.ks), reinterpret_cast<const float*>(ws + L.va), o, p,
                     L.sq_pad, L.skv_pad);
  return hipGetLastError();
}

}  // namespace mxa

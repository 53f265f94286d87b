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
#include <atomic>
#include <chrono>
#include <cstdlib>
#include <random>
#include <type_traits>

#include "attn_common.hpp"
#include "norm_rope.hpp"
#include "sage_tile.inc"


namespace mxa {

namespace {

// ---------------- prologue ----------------
//
// Eager calls with Skv <= 8192 (plain prologue) run prep_kv_fused, one launch over K
// and V (below), plus prep_stats_q's Q blocks when Q is quantized here. Otherwise
// three launches (the reference uses a memset and four kernels, :433-446):
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
constexpr int kFoldNb = 32;       // statistics partials per head up to which prep_kv_quant finalizes them

// NRM >= 0: q and k are the raw projections; every row gets the per-head RMS-norm
// + RoPE of head_norm_rope (nq / nk, nr128_row with rope mode NRM) and its bf16
// rounding on the way in, so the workspace is bit-identical to head_norm_rope
// followed by the plain prologue. NRM = -1: the plain prologue.
// QG: Q scale group in rows, 16 (the reference) or 64 (one scale per 64-token
// block, written to each of its four 16-row entries so the attention kernel is unchanged).
// D: head dimension, 64 or 128 (the fused norm/rope variants: 128 only).
template <int D, int NRM, int QG>
__global__ void __launch_bounds__(256) prep_stats_q(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                    const uint16_t* __restrict__ v, mx_attn_params p, int nb,
                                                    float qmult, int64_t sq_pad, float* __restrict__ part,
                                                    int8_t* __restrict__ qi, float* __restrict__ qs, NormRope nq,
                                                    NormRope nk) {
  __shared__ __align__(16) uint16_t kt[kStatChunk * D];
  __shared__ __align__(16) uint16_t vt_[kStatChunk * D];
  static_assert(D == 64 || D == 128, "head dimension 64 or 128");
  static_assert(NRM < 0 || D == 128, "the fused norm/rope prologue is built for D = 128");
  const int tid = threadIdx.x, nstat = p.Hkv * nb;
  if (int(blockIdx.x) < nstat) {
    // ---- K sum / V abs-max over tokens [b*256, min(b*256+256, Skv)) of head h ----
    const int h = blockIdx.x / nb, b = blockIdx.x % nb;
    const int64_t t0 = int64_t(b) * kStatTok;
    const int64_t t1 = t0 + kStatTok < p.Skv ? t0 + kStatTok : p.Skv;
    float sum = 0.f, am = 0.f;
    // sequential per-channel sum (K, token order) / abs-max (V) of the chunk staged in LDS
    auto fold = [&](int rows) __attribute__((always_inline)) {
      if (tid < D) {
#pragma unroll 16
        for (int r = 0; r < rows; ++r) sum += bf2f(kt[r * D + tid]);  // sequential, token order
      } else if (tid < 2 * D) {
        const int d = tid - D;
#pragma unroll 16
        for (int r = 0; r < rows; ++r) am = fmaxf(am, fabsf(bf2f(vt_[r * D + d])));
      }
    };
    if constexpr (NRM < 0) {
      // every load of a chunk in flight before the first LDS store, and the next chunk's
      // loads in flight while this one is folded (rows past a chunk's end are not
      // loaded; their LDS rows are never read)
      constexpr int NL = kStatChunk * (D / 8) / 256;
      u32x4 kr[NL], vr[NL];
      auto load = [&](int64_t c0, int rows) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NL; ++u) {
          const int i = tid + 256 * u, r = i / (D / 8), c = (i % (D / 8)) * 8;
          const int64_t g = (c0 + r) * p.kv_stride + int64_t(h) * D + c;
          kr[u] = vr[u] = u32x4{0, 0, 0, 0};
          if (r < rows) {
            kr[u] = *reinterpret_cast<const u32x4*>(k + g);
            vr[u] = *reinterpret_cast<const u32x4*>(v + g);
          }
        }
      };
      const int nch = int((t1 - t0 + kStatChunk - 1) / kStatChunk);  // 1 or 2
      load(t0, int(t1 - t0 < kStatChunk ? t1 - t0 : kStatChunk));
      for (int ch = 0; ch < nch; ++ch) {
        const int64_t c0 = t0 + int64_t(ch) * kStatChunk;
        const int rows = int(t1 - c0 < kStatChunk ? t1 - c0 : kStatChunk);
#pragma unroll
        for (int u = 0; u < NL; ++u) {
          const int i = tid + 256 * u, r = i / (D / 8), c = (i % (D / 8)) * 8;
          *reinterpret_cast<u32x4*>(&kt[r * D + c]) = kr[u];
          *reinterpret_cast<u32x4*>(&vt_[r * D + c]) = vr[u];
        }
        __syncthreads();
        if (ch + 1 < nch) load(c0 + kStatChunk, int(t1 - c0 - kStatChunk < kStatChunk ? t1 - c0 - kStatChunk
                                                                                       : kStatChunk));
        fold(rows);
        __syncthreads();
      }
    } else {
      for (int64_t c0 = t0; c0 < t1; c0 += kStatChunk) {
        const int rows = int(t1 - c0 < kStatChunk ? t1 - c0 : kStatChunk);
        {
          // K rows normalised on the way into LDS: one row per 16 lanes, 16 per pass
          // (all eight rows of a lane group loaded before any is normalised)
          const int lane = tid & 63, c = (lane & 15) * 8;
          constexpr int RPG = kStatChunk / 16;  // rows per 16-lane group
          u32x4 raw[RPG];
#pragma unroll
          for (int u = 0; u < RPG; ++u) {
            const int r = u * 16 + (tid >> 4);
            raw[u] = u32x4{0, 0, 0, 0};
            if (r < rows) raw[u] = *reinterpret_cast<const u32x4*>(k + (c0 + r) * p.kv_stride + int64_t(h) * D + c);
          }
#pragma unroll
          for (int u = 0; u < RPG; ++u) {
            const int r = u * 16 + (tid >> 4);
            float x[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = bf2f(uint16_t(raw[u][j >> 1] >> ((j & 1) * 16)));
            nr128_row<NRM>(x, c0 + r, r < rows, nk, lane);
            if (r < rows) *reinterpret_cast<u32x4*>(&kt[r * D + c]) = pack8_bf16(x);
          }
          for (int i = tid; i < rows * (D / 8); i += 256) {
            const int r = i / (D / 8), cc = (i % (D / 8)) * 8;
            *reinterpret_cast<u32x4*>(&vt_[r * D + cc]) =
                *reinterpret_cast<const u32x4*>(v + (c0 + r) * p.kv_stride + int64_t(h) * D + cc);
          }
        }
        __syncthreads();
        fold(rows);
        __syncthreads();
      }
    }
    if (tid < D) part[(int64_t(h) * nb + b) * D + tid] = sum / float(p.Skv);
    else if (tid < 2 * D) part[int64_t(p.Hkv) * nb * D + (int64_t(h) * nb + b) * D + (tid - D)] = am;
    return;
  }
  // ---- Q: one 16-row group per wave; lane owns D / 32 chunks of 8 channels ----
  const int wave = tid >> 6, lane = tid & 63;
  const int64_t gid = (int64_t(blockIdx.x) - nstat) * 4 + wave;  // group index over (head, group)
  const int ng = int(sq_pad / 16);
  if (gid >= int64_t(p.Hq) * ng) return;
  const int h = int(gid / ng), grp = int(gid % ng);
  constexpr int NCH = D / 32, CPR = D / 8;  // chunks per lane, chunks per row
  float x[NCH][8], am = 0.f;
  u32x4 raw[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int ci = lane + i * 64, r = ci / CPR, c = (ci % CPR) * 8;
    const int64_t row = int64_t(grp) * 16 + r;
    raw[i] = u32x4{0, 0, 0, 0};
    if (row < p.Sq) raw[i] = *reinterpret_cast<const u32x4*>(q + row * p.q_stride + int64_t(h) * D + c);
  }
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int64_t row = int64_t(grp) * 16 + (lane + i * 64) / CPR;
#pragma unroll
    for (int j = 0; j < 8; ++j) x[i][j] = bf2f(uint16_t(raw[i][j >> 1] >> ((j & 1) * 16)));
    // row r of the group on lanes 16(r&3) .. +15: the 16-lane layout of nr128_row
    if constexpr (NRM >= 0) nr128_row<NRM>(x[i], row, row < p.Sq, nq, lane);
#pragma unroll
    for (int j = 0; j < 8; ++j) am = fmaxf(am, fabsf(x[i][j]));
  }
  am = wave_max(am);
  if constexpr (QG == 64) {  // the work-group's four waves hold the 64-row block
    __shared__ float wmax[4];
    if (lane == 0) wmax[wave] = am;
    __syncthreads();
    am = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  }
  const float inv = am > 0.f ? 127.f / am : 0.f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int ci = lane + i * 64, r = ci / CPR, c = (ci % CPR) * 8;
    *reinterpret_cast<u32x2*>(qi + (int64_t(h) * sq_pad + int64_t(grp) * 16 + r) * D + c) = quant8(x[i], inv);
  }
  if (lane == 0) qs[int64_t(h) * (sq_pad / 16) + grp] = am / 127.f * qmult;
}

// kmean / vamax of one head from the statistics partials: the sum in ascending
// block order from 0.f, the max (prep_finalize's arithmetic, shared so the fused
// path is bit-identical).
template <int D>
__device__ __forceinline__ void finalize_channel(const float* ps, const float* pa, int nb, float& s, float& am) {
  constexpr int B = 16;
  s = 0.f;
  am = 0.f;
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
}

// kmean = sum of the partials in ascending block order from 0.f; vamax = max.
template <int D>
__global__ void __launch_bounds__(D) prep_finalize(mx_attn_params p, int nb, const float* __restrict__ part,
                                                   float* __restrict__ km, float* __restrict__ va,
                                                   int* __restrict__ cnt, int ncnt) {
  const int h = blockIdx.x, d = threadIdx.x;
  if (h == 0)  // arrival counters of the attention kernel's split units start at zero
    for (int i = d; i < ncnt; i += D) cnt[i] = 0;
  const float* ps = part + int64_t(h) * nb * D + d;
  float s, am;
  finalize_channel<D>(ps, ps + int64_t(p.Hkv) * nb * D, nb, s, am);
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
// chunk tid % (D/8) (8 channels) of the D/32 consecutive keys from (tid / (D/8)) D/32.
// fold_nb > 0: prep_finalize is folded in (short sequences, few partials): every
// work-group sums its head's fold_nb partials itself, work-groups of tile 0 store
// the head's km / va, and work-group (0, 0) zeroes the attention kernel's split
// counters. fold_nb == 0: km / va come from prep_finalize.
template <int D, int NRM>
__global__ void __launch_bounds__(256) prep_kv_quant(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                     mx_attn_params p, int64_t skv_pad, float* __restrict__ km,
                                                     float* __restrict__ va, int8_t* __restrict__ ki,
                                                     float* __restrict__ ks, uint8_t* __restrict__ vt, NormRope nk,
                                                     int fold_nb, const float* __restrict__ part,
                                                     int* __restrict__ cnt, int ncnt, u32x4* __restrict__ tab) {
  __shared__ __align__(16) uint8_t tile[D][kKvPad + 16];
  __shared__ float red[4];
  __shared__ float kms[D], vas[D];
  static_assert(D == 64 || D == 128, "head dimension 64 or 128");
  static_assert(NRM < 0 || D == 128, "the fused norm/rope prologue is built for D = 128");
  constexpr int CPR = D / 8, RPP = 256 / CPR, NI = kKvPad / RPP;  // chunks per row, rows per pass, passes
  const int h = blockIdx.y, k0 = blockIdx.x * kKvPad, tid = threadIdx.x;
  const int c = (tid % CPR) * 8, kr0 = (tid / CPR) * NI;  // channels c..c+7 of keys kr0..kr0+NI-1
  const float* kmh = km + h * D;
  const float* vah = va + h * D;
  if (fold_nb > 0) {
    if (tid < D) {
      const float* ps = part + int64_t(h) * fold_nb * D + tid;
      float sm, am;
      finalize_channel<D>(ps, ps + int64_t(p.Hkv) * fold_nb * D, fold_nb, sm, am);
      kms[tid] = sm;
      vas[tid] = am;
      if (blockIdx.x == 0) {
        km[h * D + tid] = sm;
        va[h * D + tid] = am;
      }
    }
    if (blockIdx.x == 0 && blockIdx.y == 0)
      for (int i = tid; i < ncnt; i += 256) cnt[i] = 0;
    __syncthreads();
    kmh = kms;
    vah = vas;
  }
  float mean[8], vsc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    mean[j] = kmh[c + j];
    const float a = vah[c + j];
    vsc[j] = a > 0.f ? 448.f / a : 0.f;
  }
  u32x4 kraw[NI], vraw[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int64_t row = k0 + kr0 + i;
    kraw[i] = vraw[i] = u32x4{0, 0, 0, 0};
    if (row < p.Skv) {
      const int64_t g = row * p.kv_stride + int64_t(h) * D + c;
      kraw[i] = *reinterpret_cast<const u32x4*>(k + g);
      vraw[i] = *reinterpret_cast<const u32x4*>(v + g);
    }
  }
  // K: x' = bf16(x) - mean (rows >= Skv are 0), amax over the tile
  float x[NI][8], am = 0.f;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int64_t row = k0 + kr0 + i;
    const bool ok = row < p.Skv;
#pragma unroll
    for (int j = 0; j < 8; ++j) x[i][j] = bf2f(uint16_t(kraw[i][j >> 1] >> ((j & 1) * 16)));
    if constexpr (NRM >= 0) nr128_row<NRM>(x[i], row, ok, nk, threadIdx.x & 63);  // row per 16 lanes
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x[i][j] = ok ? x[i][j] - mean[j] : 0.f;
      am = fmaxf(am, fabsf(x[i][j]));
    }
  }
  // V -> e4m3 into the transposed LDS tile while the K amax reduces: the thread's NI
  // consecutive keys of each of its 8 channels go out as one NI-byte LDS write; the
  // 16-byte key chunk q of channel row d sits at chunk q ^ ((d >> 4) & 3), which with
  // the 80-byte row pitch spreads a wave's writes over 32 banks
  static_assert(NI == 4 || NI == 2, "keys per thread");
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float f[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const bool ok = k0 + kr0 + i < p.Skv && vsc[j] > 0.f;
      f[i] = ok ? bf2f(uint16_t(vraw[i][j >> 1] >> ((j & 1) * 16))) * vsc[j] : 0.f;
    }
    const int d = c + j;
    uint8_t* dst = &tile[d][16 * ((kr0 >> 4) ^ ((d >> 4) & 3)) + (kr0 & 15)];
    if constexpr (NI == 4)
      *reinterpret_cast<uint32_t*>(dst) = e4m3x2_sat(f[0], f[1]) | (e4m3x2_sat(f[2], f[3]) << 16);
    else
      *reinterpret_cast<uint16_t*>(dst) = uint16_t(e4m3x2_sat(f[0], f[1]));
  }
  am = wave_max(am);
  if ((tid & 63) == 0) red[tid >> 6] = am;
  __syncthreads();
  am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float inv = am > 0.f ? 127.f / am : 0.f;
#pragma unroll
  for (int i = 0; i < NI; ++i)
    *reinterpret_cast<u32x2*>(ki + (int64_t(h) * skv_pad + k0 + kr0 + i) * D + c) = quant8(x[i], inv);
  if (tid == 0) ks[int64_t(h) * (skv_pad / kKvPad) + blockIdx.x] = am / 127.f * 1.f;
  // tile table of the attention kernel: liveness bits of the tile's 64 keys (mask and
  // tail) and its K scale, negated when some key is dead (the kernel's loop branches on
  // that sign and uses the magnitude)
  if (tid < 64) {
    const int64_t key = k0 + tid;
    const bool live = key < p.Skv && (!p.kv_valid || p.kv_valid[key]);
    const uint64_t bits = __ballot(live);
    if (tid == 0)
      tab[int64_t(h) * (skv_pad / kKvPad + 1) + blockIdx.x] =
          u32x4{uint32_t(bits), uint32_t(bits >> 32), __float_as_uint(bits == ~0ull ? am / 127.f : -(am / 127.f)),
                0u};
  }
  // V^T rows: channel d, 64 keys = 4 x 16 bytes
  for (int i = tid; i < D * (kKvPad / 16); i += 256) {
    const int d = i / (kKvPad / 16), u = i % (kKvPad / 16);
    *reinterpret_cast<u32x4*>(vt + (int64_t(h) * D + d) * skv_pad + k0 + u * 16) =
        *reinterpret_cast<const u32x4*>(&tile[d][16 * (u ^ ((d >> 4) & 3))]);
  }
}

// ---------------- one-pass K/V prologue ----------------
//
// prep_kv_fused replaces prep_stats_q's K/V blocks, prep_finalize and prep_kv_quant
// with one launch that reads K and V once: work-group (h, b) loads its 256-token
// block of K and V into registers, publishes the block's statistics partial
// (sequential K sum / Skv, V abs-max) and a ready flag, waits until its head's
// K mean and V abs-max are known, and quantizes the block from its registers.
// Same arithmetic as the three-launch path (bit-identical workspace).
//
// Flags: ws.flg holds one 64-bit word per (head, block); a word is
// "set" when it equals the call's epoch, a per-process counter that never repeats
// (and is never 0), so no flag needs clearing before a call and a workspace reused
// across calls cannot satisfy a wait with an old flag. The host runs this path only
// outside stream capture: a captured launch would replay with one fixed epoch.
//
// Waiting: work-groups are dispatched in index order and a head's blocks are
// consecutive, so a head's blocks all get a slot while earlier heads drain (a head
// holds at most kFoldNb work-groups). The wait is bounded all the same: after
// kFusedWaitTicks of the 100 MHz chip clock a work-group stops waiting and computes
// every partial whose flag it has not seen from K and V in memory (the same bytes
// the missing block would write), so the kernel ends whatever the dispatch order.
//
// Every work-group sums its head's nb <= kFoldNb partials itself. Beyond that (Skv >
// 8192) the three-launch path runs: a variant in which the head's last block folded
// the partials and published them with a head flag measured no faster at 49 blocks
// per head and slower at 128 (its waiting work-groups hold slots the loads need).
//
// Memory ordering across work-groups (and XCDs, whose L2s are not coherent): partials
// and flags move with device-scope relaxed atomics (sc1 accesses, served at the
// device-coherent level); a publisher waits for its stores' acknowledgements
// (vmcnt(0)) and passes a work-group barrier before lane 0 stores the flag, and a
// reader loads the data only after the barrier that follows its flag loads.
constexpr uint64_t kFusedWaitTicks = 20000;  // 200 us
// Bound in use (mx_sage_prologue_wait_ticks changes it for tests of the recompute path).
std::atomic<uint64_t> g_fused_wait_ticks{kFusedWaitTicks};

__device__ __forceinline__ void st_dev(float* p, float x) {
  __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// True when flags f[0..n) all equal epoch; false once `ticks` of the chip clock have
// passed (ticks 0: one look). Work-group uniform; every thread must call it.
__device__ __forceinline__ bool wait_flags(const uint64_t* f, int n, uint64_t epoch, uint64_t ticks) {
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (;;) {
    bool ok = true;
    for (int j = threadIdx.x; j < n; j += blockDim.x)
      ok &= __hip_atomic_load(const_cast<uint64_t*>(f + j), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == epoch;
    if (__syncthreads_and(ok)) return true;
    const bool late = threadIdx.x == 0 && __builtin_amdgcn_s_memrealtime() - t0 >= ticks;
    if (__syncthreads_or(late)) return false;
    __builtin_amdgcn_s_sleep(2);
  }
}

// Statistics partial of block b of head h computed from K and V in memory (the
// fallback of a wait that timed out), staged through `sm` in 128-token chunks exactly
// as prep_stats_q does, stored with device-scope stores. Threads < D: K sum, D..2D-1:
// V abs-max.
template <int D>
__device__ void fused_stats_from_memory(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                        const mx_attn_params& p, int h, int b, int nb, float* part,
                                        unsigned char* sm) {
  uint16_t* kt = reinterpret_cast<uint16_t*>(sm);
  uint16_t* vt_ = kt + kStatChunk * D;
  const int tid = threadIdx.x;
  const int64_t t0 = int64_t(b) * kStatTok;
  const int64_t t1 = t0 + kStatTok < p.Skv ? t0 + kStatTok : p.Skv;
  float sum = 0.f, am = 0.f;
  for (int64_t c0 = t0; c0 < t1; c0 += kStatChunk) {
    const int rows = int(t1 - c0 < kStatChunk ? t1 - c0 : kStatChunk);
    __syncthreads();
    for (int i = tid; i < rows * (D / 8); i += blockDim.x) {
      const int r = i / (D / 8), c = (i % (D / 8)) * 8;
      const int64_t g = (c0 + r) * p.kv_stride + int64_t(h) * D + c;
      *reinterpret_cast<u32x4*>(&kt[r * D + c]) = *reinterpret_cast<const u32x4*>(k + g);
      *reinterpret_cast<u32x4*>(&vt_[r * D + c]) = *reinterpret_cast<const u32x4*>(v + g);
    }
    __syncthreads();
    if (tid < D) {
      for (int r = 0; r < rows; ++r) sum += bf2f(kt[r * D + tid]);
    } else if (tid < 2 * D) {
      for (int r = 0; r < rows; ++r) am = fmaxf(am, fabsf(bf2f(vt_[r * D + tid - D])));
    }
  }
  if (tid < D) st_dev(part + (int64_t(h) * nb + b) * D + tid, sum / float(p.Skv));
  else if (tid < 2 * D) st_dev(part + int64_t(p.Hkv) * nb * D + (int64_t(h) * nb + b) * D + (tid - D), am);
  __syncthreads();
}

// Wait for every block flag of head h (bounded), compute the partials still missing,
// and return this thread's channel of K mean / V abs-max (threads < D) summed in
// ascending block order (finalize_channel's arithmetic on device-scope loads).
template <int D>
__device__ void fused_fold(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, const mx_attn_params& p,
                           int h, int nb, float* part, const uint64_t* flg, uint64_t epoch, uint64_t ticks,
                           unsigned char* sm, bool* miss, float& s, float& am) {
  const uint64_t* fh = flg + int64_t(h) * nb;
  if (!wait_flags(fh, nb, epoch, ticks)) {
    for (int j = threadIdx.x; j < nb; j += blockDim.x)
      miss[j] = __hip_atomic_load(const_cast<uint64_t*>(fh + j), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != epoch;
    __syncthreads();
    for (int j = 0; j < nb; ++j)
      if (miss[j]) fused_stats_from_memory<D>(k, v, p, h, j, nb, part, sm);
    wait_vm();
    __syncthreads();
  }
  // the head's partials: 16-byte device-scope loads by every thread (all issued before
  // the first is used), staged in LDS, then each channel summed in ascending block order
  // (finalize_channel's arithmetic); at most kFoldNb blocks per pass
  s = 0.f;
  am = 0.f;
  float* pl = reinterpret_cast<float*>(sm);  // [2][kFoldNb][D]
  constexpr int kSc1 = 16;                    // cache policy: device scope
  const int64_t half = int64_t(p.Hkv) * nb * D;
  const __amdgpu_buffer_rsrc_t rk = buf_rsrc(part + int64_t(h) * nb * D, uint32_t(nb) * D * 4u);
  const __amdgpu_buffer_rsrc_t rv = buf_rsrc(part + half + int64_t(h) * nb * D, uint32_t(nb) * D * 4u);
  constexpr int NQ = 2 * kFoldNb * D / 4 / 512;  // 16-byte loads per thread per pass
  for (int b0 = 0; b0 < nb; b0 += kFoldNb) {
    const int nbp = nb - b0 < kFoldNb ? nb - b0 : kFoldNb;
    u32x4 x[NQ];
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int e = (int(threadIdx.x) + i * 512) * 4;  // float index in [2][kFoldNb][D]
      const int which = e / (kFoldNb * D), r = e % (kFoldNb * D);
      x[i] = u32x4{0, 0, 0, 0};
      if (r < nbp * D)
        x[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             which ? rv : rk, uint32_t(r) * 4u, uint32_t(b0) * D * 4u, kSc1));
    }
#pragma unroll
    for (int i = 0; i < NQ; ++i) *reinterpret_cast<u32x4*>(pl + (int(threadIdx.x) + i * 512) * 4) = x[i];
    __syncthreads();
    if (threadIdx.x < D)
      for (int j = 0; j < nbp; ++j) {
        s += pl[j * D + threadIdx.x];
        am = fmaxf(am, pl[kFoldNb * D + j * D + threadIdx.x]);
      }
    __syncthreads();
  }
}

// One work-group of 512 threads per (head, 256-token block): thread t owns channel
// chunk c = t % (D/8) (8 channels) of the RPT consecutive tokens from (t / (D/8)) RPT.
template <int D>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) prep_kv_fused(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                     mx_attn_params p, int nb, int64_t skv_pad,
                                                     float* __restrict__ part, float* __restrict__ km,
                                                     float* __restrict__ va, int8_t* __restrict__ ki,
                                                     float* __restrict__ ks, uint8_t* __restrict__ vt,
                                                     u32x4* __restrict__ tab, int* __restrict__ cnt, int ncnt,
                                                     uint64_t* __restrict__ flg, uint64_t epoch, uint64_t wait_ticks) {
  static_assert(D == 64 || D == 128, "head dimension 64 or 128");
  constexpr int NT = 512, CPR = D / 8, RPT = kStatTok * CPR / NT;  // chunks per row, tokens per thread
  constexpr int TPT = kKvPad / RPT * CPR;                           // threads per 64-key tile (128)
  static_assert(TPT == 128, "layout");
  // V^T granule swizzle of channel chunk cc: D = 128 (32 granules of 8 bytes per row; a
  // 32-lane pass of 8-byte writes covers 16 chunks x 2 granules): (cc & 15) << 1; D = 64
  // (64 granules of 4 bytes; a 64-lane pass covers 8 chunks x 8 granules): cc << 3. Both
  // give every lane of a pass its own bank pair / bank and keep each 16-byte read's
  // granules adjacent and in order.
  auto vsw = [](int cc) __attribute__((always_inline)) { return D == 128 ? (cc & 15) << 1 : (cc & 7) << 3; };
  __shared__ __align__(16) unsigned char sm[kStatTok * D * 2];  // K rows, then V^T
  __shared__ float red[NT / 64][D];
  __shared__ float kms[D], vas[D];
  __shared__ bool miss[kFoldNb];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h = blockIdx.x / nb, b = blockIdx.x % nb;
  const int c = tid % CPR, r0 = (tid / CPR) * RPT;
  const int64_t t0 = int64_t(b) * kStatTok;
  const int rows = int(p.Skv - t0 < kStatTok ? p.Skv - t0 : kStatTok);
  MX_STAMP(0);

  u32x4 kr[RPT], vr[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    kr[i] = vr[i] = u32x4{0, 0, 0, 0};
    if (r0 + i < rows) {
      const int64_t g = (t0 + r0 + i) * p.kv_stride + int64_t(h) * D + c * 8;
      kr[i] = *reinterpret_cast<const u32x4*>(k + g);
      vr[i] = *reinterpret_cast<const u32x4*>(v + g);
    }
  }
  if (blockIdx.x == 0)  // arrival counters of the attention kernel's split units start at zero
    for (int i = tid; i < ncnt; i += NT) cnt[i] = 0;

  // ---- statistics partial: K rows through LDS for the sequential per-channel sum,
  // V abs-max from registers (a max does not depend on order) ----
  // D = 128: channel-major [D][256 tokens] (16-byte chunk u of channel row d at chunk
  // u ^ ((d ^ (d >> 3)) & 15): conflict-free both for the writes, 16 channels of one
  // chunk per pass, and for the sum's reads, 16 channels' same chunk), so the sum reads
  // 8 tokens per LDS read; D = 64: token-major [256][D]
  uint16_t* kst = reinterpret_cast<uint16_t*>(sm);
  if constexpr (D == 128) {
#pragma unroll
    for (int j2 = 0; j2 < 4; ++j2)
#pragma unroll
      for (int hi = 0; hi < 2; ++hi) {
        const int d = c * 8 + j2 * 2 + hi;
        const uint32_t sel = hi ? 0x07060302u : 0x05040100u;  // high / low bf16 of each word
        u32x4 col;
#pragma unroll
        for (int m = 0; m < 4; ++m) col[m] = __builtin_amdgcn_perm(kr[2 * m + 1][j2], kr[2 * m][j2], sel);
        *reinterpret_cast<u32x4*>(sm + d * 512 + ((r0 / 8) ^ ((d ^ (d >> 3)) & 15)) * 16) = col;
      }
  } else {
#pragma unroll
    for (int i = 0; i < RPT; ++i) *reinterpret_cast<u32x4*>(&kst[(r0 + i) * D + c * 8]) = kr[i];
  }
  // |v| as bf16 bits (sign cleared) ordered as integers: a packed 16-bit max per pair
  // of channels equals the float max of |v| for every non-NaN input
  using u16x2 = __attribute__((ext_vector_type(2))) unsigned short;
  u16x2 vam[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    vam[w] = u16x2{0, 0};
#pragma unroll
    for (int i = 0; i < RPT; ++i)
      vam[w] = __builtin_elementwise_max(vam[w], __builtin_bit_cast(u16x2, uint32_t(vr[i][w] & 0x7fff7fffu)));
#pragma unroll
    for (int off = CPR; off < 64; off <<= 1)
      vam[w] = __builtin_elementwise_max(
          vam[w], __builtin_bit_cast(u16x2, uint32_t(__shfl_xor(int(__builtin_bit_cast(uint32_t, vam[w])), off))));
  }
  if (lane < CPR)
#pragma unroll
    for (int j = 0; j < 8; ++j) red[wave][c * 8 + j] = bf2f(vam[j >> 1][j & 1]);
  __syncthreads();
  MX_STAMP(1);
  if (tid < D) {
    float sum = 0.f;
    if constexpr (D == 128) {  // tokens past the block's end are zeros: adding +0 changes no sum
                               // (a sum from +0 is never -0)
      const int sw = (tid ^ (tid >> 3)) & 15;
#pragma unroll 2
      for (int u = 0; u < kStatTok / 8; ++u) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(sm + tid * 512 + (u ^ sw) * 16);
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += bf2f(uint16_t(w[e >> 1] >> ((e & 1) * 16)));  // token order
      }
    } else {
#pragma unroll 16
      for (int r = 0; r < rows; ++r) sum += bf2f(kst[r * D + tid]);  // sequential, token order
    }
    st_dev(part + (int64_t(h) * nb + b) * D + tid, sum / float(p.Skv));
  } else if (tid < 2 * D) {
    float am = 0.f;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) am = fmaxf(am, red[w][tid - D]);
    st_dev(part + int64_t(p.Hkv) * nb * D + (int64_t(h) * nb + b) * D + (tid - D), am);
  }
  wait_vm();
  __syncthreads();
  if (tid == 0)
    __hip_atomic_store(flg + int64_t(h) * nb + b, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  MX_STAMP(2);

  // ---- K mean and V abs-max of the head: every work-group folds the partials ----
  float s = 0.f, am = 0.f;
  fused_fold<D>(k, v, p, h, nb, part, flg, epoch, wait_ticks, sm, miss, s, am);
  if (b == 0 && tid < D) {
    km[h * D + tid] = s;
    va[h * D + tid] = am;
  }
  if (tid < D) {
    kms[tid] = s;
    vas[tid] = am > 0.f ? 448.f / am : 0.f;  // the channel's V scale, one division per channel
  }
  __syncthreads();  // also: every read of the K rows in sm is done
  MX_STAMP(3);

  // ---- K - mean -> INT8, one scale per 64-key tile (threads [128 tl, 128 tl + 128)) ----
  const int tl = tid / TPT;
  const int64_t key0 = t0 + tl * kKvPad;  // first key of this thread's tile
  float mean[8], vsc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) mean[j] = kms[c * 8 + j], vsc[j] = vas[c * 8 + j];
  // rows past Skv (loaded as zeros) give 0; a whole block (every block but a head's
  // last, usually) takes the version without the row test (FULL)
  const bool full = rows == kStatTok;
  auto kx = [&](int i, int j, auto fullc) __attribute__((always_inline)) {
    const float x = bf2f(uint16_t(kr[i][j >> 1] >> ((j & 1) * 16))) - mean[j];
    if constexpr (decltype(fullc)::value) return x;
    else return r0 + i < rows ? x : 0.f;
  };
  auto k_amax = [&](auto fullc) __attribute__((always_inline)) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(kx(i, j, fullc)));
    return m;
  };
  float tam = full ? k_amax(std::true_type{}) : k_amax(std::false_type{});
  tam = wave_max(tam);
  float* tred = &red[0][0];
  if (lane == 0) tred[wave] = tam;

  // ---- V -> e4m3 into the V^T tile in LDS: channel row d, RPT-byte granule of
  // tokens r0.. at granule (r0 / RPT) ^ vsw(c), which spreads a wave's
  // writes over every bank ----
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    // rows past Skv are zeros (0 * vsc = +0); a channel with no nonzero value stays 0
    float f[RPT];
    const bool live = vsc[j] > 0.f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const float x = bf2f(uint16_t(vr[i][j >> 1] >> ((j & 1) * 16))) * vsc[j];
      f[i] = live ? x : 0.f;
    }
    const int d = c * 8 + j, gi = (r0 / RPT) ^ vsw(c);
    unsigned char* dst = sm + d * kStatTok + gi * RPT;
    if constexpr (RPT == 8)
      *reinterpret_cast<u32x2*>(dst) = u32x2{e4m3x2_sat(f[0], f[1]) | (e4m3x2_sat(f[2], f[3]) << 16),
                                             e4m3x2_sat(f[4], f[5]) | (e4m3x2_sat(f[6], f[7]) << 16)};
    else
      *reinterpret_cast<uint32_t*>(dst) = e4m3x2_sat(f[0], f[1]) | (e4m3x2_sat(f[2], f[3]) << 16);
  }
  __syncthreads();
  tam = fmaxf(tred[2 * tl], tred[2 * tl + 1]);
  const float inv = tam > 0.f ? 127.f / tam : 0.f;
  if (key0 < skv_pad) {
    auto k_store = [&](auto fullc) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = kx(i, j, fullc);
        *reinterpret_cast<u32x2*>(ki + (int64_t(h) * skv_pad + t0 + r0 + i) * D + c * 8) = quant8(x, inv);
      }
    };
    if (full) k_store(std::true_type{});
    else k_store(std::false_type{});
    if ((tid & (TPT - 1)) == 0) ks[int64_t(h) * (skv_pad / kKvPad) + key0 / kKvPad] = tam / 127.f * 1.f;
    // tile table entry (as prep_kv_quant): liveness bits, K scale negated when a key is dead
    if ((tid & (TPT - 1)) < 64) {
      const int64_t key = key0 + lane;
      const bool live = key < p.Skv && (!p.kv_valid || p.kv_valid[key]);
      const uint64_t bits = __ballot(live);
      if (lane == 0)
        tab[int64_t(h) * (skv_pad / kKvPad + 1) + key0 / kKvPad] =
            u32x4{uint32_t(bits), uint32_t(bits >> 32),
                  __float_as_uint(bits == ~0ull ? tam / 127.f : -(tam / 127.f)), 0u};
    }
  }
  // ---- V^T rows: channel d, the block's keys below skv_pad, 16 bytes per thread ----
  const int nkeys = int(skv_pad - t0 < kStatTok ? skv_pad - t0 : kStatTok);
  for (int i = tid; i < D * (kStatTok / 16); i += NT) {
    const int d = i / (kStatTok / 16), u = i % (kStatTok / 16);
    if (u * 16 >= nkeys) continue;
    const int gi = (u * (16 / RPT)) ^ vsw(d >> 3);
    *reinterpret_cast<u32x4*>(vt + (int64_t(h) * D + d) * skv_pad + t0 + u * 16) =
        *reinterpret_cast<const u32x4*>(sm + d * kStatTok + gi * RPT);
  }
#ifdef MX_STAMPS
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  MX_STAMP(4);
#endif
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
// Schedule: lockstep, every wave runs S -> softmax -> P*V per tile. The softmax
// is the larger share of the work here (the INT8/FP8 MFMAs take half the cycles
// of BF16 ones) and bounds the kernel. A ping-pong schedule like the BF16
// kernel's was measured ~10% slower: a wave running the softmax alone on a SIMD
// does not get the dual issue of fp32 adds/FMAs that two interleaved waves get,
// and a neighbouring MFMA wave slows it by a further 20-30%.

constexpr int KT = 64;
constexpr int kPipeD = 128;               // head dimension of sage_attn_pipe
constexpr int KTILEB = KT * kPipeD;       // 8 KB int8 K tile (D = 128)
constexpr int VTILEB = kPipeD * KT;       // 8 KB fp8 V^T tile (D = 128)
// Split partial of one work-group of NW waves at head dimension d (see sage_plan), in
// 4-byte words: o = acc / (448 l) in fp16 as [NW waves][d/16 groups of 8][64 lanes],
// then m and l as [NW waves][64 lanes][2] floats.
constexpr int split_acc(int nw, int d) { return nw * (d / 16) * 64 * 4; }
constexpr int split_floats(int nw, int d) { return split_acc(nw, d) + nw * 64 * 2; }
constexpr int kMaxParts = 4;  // bounds the merge's reads (parts x 132 KB per unit)
struct SageSplit {
  int full, parts;  // work-groups [0, full) run whole units; the rest run one of `parts` key ranges
  float* part;      // partials, split_floats(NW, D) per split work-group
  int* cnt;         // arrival counter per split unit
};
constexpr float kSageHeadroom = 3.f;
constexpr int kScoreBias = 0x4B400000;  // bits of 12582912.0f = 1.5 * 2^23
constexpr i32x16 kScoreBias16 = {kScoreBias, kScoreBias, kScoreBias, kScoreBias, kScoreBias, kScoreBias,
                                 kScoreBias, kScoreBias, kScoreBias, kScoreBias, kScoreBias, kScoreBias,
                                 kScoreBias, kScoreBias, kScoreBias, kScoreBias};
constexpr int kSageStages = 2;  // K/V stages of sage_attn_gen (3 and 4 measured no faster)

// Online-softmax step of one lane over the 32 biased int32 scores of a tile
// (reference attention_fp8.cu:306-345): integer row max, sc = qs * ks, one FMA into
// exp2, P packed to e4m3 four at a time (byte j of the 32-byte B operand is key
// 32h + j, j = kb*16 + ii), l over the unquantized values. Dead keys (mask, tail)
// get the bits of -inf: below every biased score as an integer (so the integer max
// skips them) and, as a float, exp2(fma(-inf, sc, nm)) = 0 exactly for sc > 0 (sc is
// clamped to >= 1e-30, which moves no live exponent). The max and the sum are
// trees and the 32 exponentials are independent, so a wave running this alone
// (ping-pong) is bound by VALU throughput rather than by dependency latency.
// Returns alpha, the rescale factor of the running output.
constexpr int kDead = int(0xFF800000u);
__device__ __forceinline__ float sage_softmax(i32x16 (&s)[2], uint64_t live, int h, float sc, float& m, float& l,
                                              i32x8& pf) {
  if (live != ~0ull) {
    // this lane's 32 keys are bits 32h .. 32h+31: select the word once, then every
    // test is a compile-time bit position (no per-lane mask registers)
    const uint32_t lw = h ? uint32_t(live >> 32) : uint32_t(live);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int ii = 0; ii < 16; ++ii)
        if (!((lw >> (kb * 16 + ii)) & 1u)) s[kb][ii] = kDead;
  }
  auto S = [&](int i) __attribute__((always_inline)) { return s[i >> 4][i & 15]; };
  int a[11];
#pragma unroll
  for (int i = 0; i < 10; ++i) a[i] = max(max(S(3 * i), S(3 * i + 1)), S(3 * i + 2));
  a[10] = max(S(30), S(31));
  const int b0 = max(max(a[0], a[1]), a[2]), b1 = max(max(a[3], a[4]), a[5]);
  const int b2 = max(max(a[6], a[7]), a[8]), b3 = max(a[9], a[10]);
  int im = max(max(b0, b1), max(b2, b3));
  im = max(im, other_half_i(im));
  const float tmax = im == kDead ? -__builtin_inff() : float(im - kScoreBias) * sc;
  const float mnew = tmax > m + kSageHeadroom ? tmax : m;
  const float alpha = m == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(m - mnew);
  m = mnew;
  // exponent = (12582912 + s)*sc + nm with nm = (log2 448 - H - m) - 12582912*sc
  // (reference attention_fp8.cu:331, :337, plus the headroom H)
  const float nm =
      mnew == -__builtin_inff() ? -__builtin_inff() : (kLog2_448 - kSageHeadroom - mnew) - 12582912.f * sc;
  float e[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) e[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(__int_as_float(S(i)), sc, nm));
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const uint32_t lo = uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(e[4 * w], e[4 * w + 1], 0, false));
    pf[w] = __builtin_amdgcn_cvt_pk_fp8_f32(e[4 * w + 2], e[4 * w + 3], int(lo), true);
  }
#pragma unroll
  for (int w = 16; w >= 1; w >>= 1)
#pragma unroll
    for (int i = 0; i < w; ++i) e[i] += e[i + w];
  const float ts = e[0] + other_half(e[0]);
  l = l * alpha + ts;
  return alpha;
}

// Score row m of key block kb -> key within the 64-key tile.
__device__ __forceinline__ int kperm(int kb, int m) {
  return ((m >> 2) & 1) * 32 + kb * 16 + (m >> 3) * 4 + (m & 3);
}

// DMA of one tile (K and V^T, D/16 ops of 1 KB each) by the eight waves of sage_attn_gen;
// K op j: rows (j&1)*32 + lane/2 of d-chunk j/2 (16-byte half XOR row bit 5); V^T op j:
// channel rows j*16 + lane/4 (16-byte chunk XOR ((row >> 2) & 3)). D = 128: wave w
// issues K op w and V^T op w; D = 64: waves 0..3 issue K op w, waves 4..7 V^T op w-4.
// Per-head buffer resources; the per-lane part of each address is loop-invariant (it
// depends on j only through j&1 == w&1), the tile and op parts are scalar.
template <int D>
struct SageAddr {
  __amdgpu_buffer_rsrc_t rk, rv;
  uint32_t lk, lv;  // per-lane byte offsets
};
template <int D>
__device__ __forceinline__ SageAddr<D> sage_addr(const int8_t* ki, const uint8_t* vt, int kvh, int64_t skv_pad,
                                                 int wave, int lane) {
  SageAddr<D> a;
  a.rk = buf_rsrc(ki + int64_t(kvh) * skv_pad * D, uint32_t(skv_pad * D));
  a.rv = buf_rsrc(vt + int64_t(kvh) * D * skv_pad, uint32_t(skv_pad * D));
  const int krow = (wave & 1) * 32 + (lane >> 1);
  a.lk = uint32_t(krow * D + (((lane & 1) ^ ((krow >> 5) & 1)) << 4));
  const int vrow = lane >> 2;  // + j*16: scalar part (does not change the XOR term)
  a.lv = uint32_t(vrow) * uint32_t(skv_pad) + uint32_t(((lane & 3) ^ ((vrow >> 2) & 3)) << 4);
  return a;
}
// DMA ops per wave per tile.
template <int D>
constexpr int sage_ops_per_wave() { return D / 64; }
// K tile tk into kdst and V^T tile tv into vdst.
template <int D>
__device__ __forceinline__ void sage_load_tile(const SageAddr<D>& a, int tk, int tv, unsigned char* kdst,
                                               unsigned char* vdst, int wave, int64_t skv_pad) {
  auto kop = [&](int j) __attribute__((always_inline)) {
    buf2lds16(a.rk, a.lk, uint32_t((j >> 1) * 32 + tk * (KT * D)), (MXA_LDS void*)(kdst + j * 1024));
  };
  auto vop = [&](int j) __attribute__((always_inline)) {
    buf2lds16(a.rv, a.lv, uint32_t(j * 16) * uint32_t(skv_pad) + uint32_t(tv * KT), (MXA_LDS void*)(vdst + j * 1024));
  };
  if constexpr (D == 128) {
    kop(wave);
    vop(wave);
  } else {
    if (wave < 4) kop(wave);
    else vop(wave - 4);
  }
}

// End of a work-group: a split part publishes its normalised output o = acc / (448 l)
// in fp16 (|o| <= 448(1 + 2^-4): a weighted mean of e4m3 values) with (m, l) and
// returns unless it is the last of its unit to arrive, which merges every part; then
// O = acc * vamax[d] / (448 l) -> bf16 for this lane's query row.
template <int NW, int D>
__device__ __forceinline__ void sage_finish(f32x16 (&acc)[D / 32], float m, float l, int part, int su, const SageSplit& sp,
                                            int wave, int lane, int row, const mx_attn_params& p,
                                            const float* __restrict__ vah, int head, uint16_t* __restrict__ o,
                                            unsigned char* stage = nullptr) {
  const int h = lane >> 5;
  if (part >= 0) {
    // Split unit: publish (o, m, l), then the last part to arrive merges all parts.
    // The partials move with device-scope (sc1) buffer accesses, which bypass the
    // XCDs' non-coherent L2s for these lines only; a device-scope fence would write
    // back and invalidate a whole L2 and with it every other work-group's K/V.
    constexpr int kSc1 = 16;  // cache policy: device scope
    constexpr int kSplitAcc = split_acc(NW, D), kSplitFloats = split_floats(NW, D);
    const uint32_t unit_bytes = uint32_t(sp.parts) * kSplitFloats * 4;
    const __amdgpu_buffer_rsrc_t rp = buf_rsrc(sp.part + int64_t(su) * sp.parts * kSplitFloats, unit_bytes);
    const uint32_t lacc = uint32_t(wave * (D / 16) * 64 + lane) * 16u;    // + j * 1024 for 8-half group j
    const uint32_t lml = uint32_t(kSplitAcc + (wave * 64 + lane) * 2) * 4u;
    const uint32_t mine = uint32_t(part) * kSplitFloats * 4u;
    const float inv = l > 0.f ? 1.f / (448.f * l) : 0.f;
    auto h2 = [](float a, float b) __attribute__((always_inline)) {
      return uint32_t(__builtin_bit_cast(uint16_t, _Float16(a))) |
             (uint32_t(__builtin_bit_cast(uint16_t, _Float16(b))) << 16);
    };
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {  // group j: acc[j / 2][(j & 1) * 8 .. + 7]
      const f32x16& a = acc[j >> 1];
      const int b = (j & 1) * 8;
      store_b128_sc1(u32x4{h2(a[b] * inv, a[b + 1] * inv), h2(a[b + 2] * inv, a[b + 3] * inv),
                           h2(a[b + 4] * inv, a[b + 5] * inv), h2(a[b + 6] * inv, a[b + 7] * inv)},
                     rp, lacc + uint32_t(j) * 1024u, mine);
    }
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{m, l}), rp, lml, mine, kSc1);
    // Publication order without a release fence: every lane waits until its sc1
    // stores are acknowledged by the device-coherent level (vmcnt(0)), the barrier
    // orders all lanes before lane 0's arrival atomic (agent scope, performed at that
    // same level), and the merging work-group reads the partials only after it has
    // seen the last arrival (its loads are issued after the barrier that follows the
    // atomic, and sc1 loads bypass the non-coherent L2, so no stale line can be hit).
    // An acq_rel atomic would add an L2 writeback + invalidate of the whole XCD.
    wait_vm();
    __shared__ int last;
    __syncthreads();
    if (threadIdx.x == 0) {
      const int prev = __hip_atomic_fetch_add(sp.cnt + su, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = prev == sp.parts - 1;
      if (last) __hip_atomic_store(sp.cnt + su, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next call
    }
    __syncthreads();
    if (!last) return;
    // merge in part order (every part read back, this one's included, so the result
    // does not depend on which part arrived last): M = max m_i, w_i = 2^(m_i - M),
    // c_i = l_i w_i, l = sum c_i, acc = sum (448 c_i) o_i
    float mi[8], li[8];
    float mm = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i >= sp.parts) break;
      const f32x2 ml = __builtin_bit_cast(
          f32x2, __builtin_amdgcn_raw_buffer_load_b64(rp, lml, uint32_t(i) * kSplitFloats * 4u, kSc1));
      mi[i] = ml[0];
      li[i] = ml[1];
      mm = fmaxf(mm, ml[0]);
    }
    l = 0.f;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) acc[db] = f32x16{};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i >= sp.parts) break;
      const float wi = mm == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(mi[i] - mm);
      const float ci = li[i] * wi;
      l += ci;
      const float c448 = 448.f * ci;
      u32x4 x[D / 16];
#pragma unroll
      for (int j = 0; j < D / 16; ++j)
        x[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            rp, lacc + uint32_t(j) * 1024u, uint32_t(i) * kSplitFloats * 4u, kSc1));
#pragma unroll
      for (int j = 0; j < D / 16; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint16_t bits = uint16_t(x[j][e >> 1] >> ((e & 1) * 16));
          acc[j >> 1][(j & 1) * 8 + e] += c448 * float(__builtin_bit_cast(_Float16, bits));
        }
    }
  }
  // ---- epilogue: O = acc * vamax[d] / (448 l) -> bf16 ----
  // Through LDS when the caller lends a staging buffer (NW * 32 rows x D bf16) and the
  // output allows 16-byte row stores: each wave writes its 32 x D block into its region
  // (16-byte chunks of row n XOR-swizzled by n), then every lane stores 16 contiguous
  // bytes, 1 KB of whole rows per instruction instead of 4-byte pieces of 32 rows.
  if (stage && (reinterpret_cast<uintptr_t>(o) & 15) == 0 && (p.o_stride & 7) == 0) {
    constexpr int CH = D / 8, RB = D * 2;
    const int n = lane & 31;
    const float inv = l > 0.f ? 1.f / (448.f * l) : 0.f;
    MXA_LDS unsigned char* wb = (MXA_LDS unsigned char*)stage + wave * 32 * RB;
    __syncthreads();  // every wave is done with the buffer (the tile loop's K ring)
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + g * 8 + h * 4;
        const f32x4 sv = *reinterpret_cast<const f32x4*>(vah + d);
        const int phys = (db * 4 + g) ^ (n & (CH - 1));
        *reinterpret_cast<MXA_LDS u32x2*>(wb + n * RB + phys * 16 + h * 8) =
            u32x2{pack_bf16x2(acc[db][g * 4] * sv[0] * inv, acc[db][g * 4 + 1] * sv[1] * inv),
                  pack_bf16x2(acc[db][g * 4 + 2] * sv[2] * inv, acc[db][g * 4 + 3] * sv[3] * inv)};
      }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const int row0 = row - n;
#pragma unroll
    for (int i = 0; i < 32 * CH / 64; ++i) {
      const int idx = i * 64 + lane, r = idx / CH, c = idx % CH;
      const u32x4 val = *reinterpret_cast<const MXA_LDS u32x4*>(wb + r * RB + ((c ^ (r & (CH - 1))) * 16));
      if (row0 + r < p.Sq) *reinterpret_cast<u32x4*>(o + int64_t(row0 + r) * p.o_stride + head * D + c * 8) = val;
    }
    return;
  }
  if (row < p.Sq) {
    const float inv = l > 0.f ? 1.f / (448.f * l) : 0.f;
    uint16_t* dst = o + int64_t(row) * p.o_stride + head * D + h * 4;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
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

template <int D, int NS>
__global__ void __launch_bounds__(512, 1)
sage_attn_gen(const int8_t* __restrict__ qi, const int8_t* __restrict__ ki, const uint8_t* __restrict__ vt,
               const float* __restrict__ qs, const float* __restrict__ ks, const float* __restrict__ va,
               uint16_t* __restrict__ o, mx_attn_params p, int64_t sq_pad, int64_t skv_pad, SageSplit sp) {
  constexpr int NW = 8, QT = NW * 32, OPS = sage_ops_per_wave<D>(), NC = D / 32;
  constexpr int KTB = KT * D, STAGEB = 2 * KT * D;  // K tile, then V^T tile
  static_assert(NS >= 2 && NS <= 4, "2..4 stages");
  static_assert(D == 64 || D == 128, "head dimension 64 or 128");
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
  const int nkt = (p.Skv + KT - 1) / KT;
  // unit (head, query tile) and key-tile range [tb, nt) of this work-group
  int L, tb = 0, nt = nkt, su = 0, part = -1;
  if (int(blockIdx.x) < sp.full) {
    L = xcd_remap(blockIdx.x, sp.full);
  } else {
    // part-major order (part 0 of every split unit, then part 1, ...), XCD-grouped:
    // each XCD runs a contiguous run of that order, i.e. one key range of consecutive
    // units (mostly one or two heads), so its L2 holds the K/V^T tiles they share
    // (unit su on XCD su % 8 spread every head over all eight L2s: 3.3x the
    // algorithmic HBM bytes)
    const int nsu = (int(gridDim.x) - sp.full) / sp.parts;
    const int j = xcd_remap(int(blockIdx.x) - sp.full, int(gridDim.x) - sp.full);
    part = j / nsu;
    su = j - part * nsu;
    L = sp.full + su;
    tb = int(int64_t(part) * nkt / sp.parts);
    nt = int(int64_t(part + 1) * nkt / sp.parts);
  }
  const int head = L / ntq, qtile = L % ntq;
  const int kvh = head / (p.Hq / p.Hkv);
  const int q0 = qtile * QT + wave * 32;

  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const SageAddr<D> sa = sage_addr<D>(ki, vt, kvh, skv_pad, wave_u, lane);
  auto issue = [&](int t, unsigned char* dst) __attribute__((always_inline)) {
    sage_load_tile<D>(sa, t, t, dst, dst + KTB, wave_u, skv_pad);
  };
  issue(tb, stage(std::integral_constant<int, 0>{}));
  if constexpr (NS > 2) if (tb + 1 < nt) issue(tb + 1, stage(std::integral_constant<int, 1>{}));
  if constexpr (NS > 3) if (tb + 2 < nt) issue(tb + 2, stage(std::integral_constant<int, 2>{}));

  // Q^T fragments: lane (n, h) holds 16 int8 channels 32c + 16h .. +15 of its query.
  const int row = q0 + n;  // < sq_pad (sq_pad is a multiple of QT)
  i32x4 qf[NC];
  {
    const int8_t* src = qi + (int64_t(head) * sq_pad + row) * D + h * 16;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) qf[cc] = *reinterpret_cast<const i32x4*>(src + cc * 32);
  }
  const float qscale = qs[int64_t(head) * (sq_pad / 16) + row / 16];
  const float* kscale = ks + int64_t(kvh) * (skv_pad / KT);
  build_live<NW, KT>(live_tiles, p, nkt, wave, lane);
  __syncthreads();  // bitmaps visible (once, before the pipelined loop)

  // Per-lane LDS read bases.
  const int krow = kperm(0, n);
  const int kbase = krow * 32 + ((h ^ ((krow >> 5) & 1)) << 4);
  const int vsw = (n >> 2) & 3;
  const int vbase0 = KTB + n * 64 + (((2 * h) ^ vsw) << 4);
  const int vbase1 = KTB + n * 64 + (((2 * h + 1) ^ vsw) << 4);

  f32x16 acc[NC];
#pragma unroll
  for (int db = 0; db < NC; ++db) acc[db] = f32x16{};
  float m = -__builtin_inff(), l = 0.f;

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
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const i32x4 a = *reinterpret_cast<const i32x4*>(sd + kbase + cc * 2048 + kb * 512);
        // accumulate on top of the bias 0x4B400000: the float with those bits + s is
        // exactly 12582912 + s (|s| < 2^22), so no int->float conversion is needed
        s[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, qf[cc], cc == 0 ? kScoreBias16 : s[kb], 0, 0, 0);
      }
    if constexpr (D == 128) {
      __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (j == 1 || j == 4) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        if (j < 5) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }

    i32x8 pf;
    const float alpha = sage_softmax(s, live, h, fmaxf(qscale * ksc, 1e-30f), m, l, pf);
    if (!__all(alpha == 1.f)) {
#pragma unroll
      for (int db = 0; db < NC; ++db) acc[db] *= alpha;
    }

    // ---- O^T += V^T P^T (e4m3 x e4m3 -> fp32) ----
#pragma unroll
    for (int db = 0; db < NC; ++db) {
      const i32x4 a0 = *reinterpret_cast<const i32x4*>(sd + vbase0 + db * 2048);
      const i32x4 a1 = *reinterpret_cast<const i32x4*>(sd + vbase1 + db * 2048);
      const i32x8 a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
      acc[db] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, pf, acc[db], 0, 0, 0, 0, 0, 0);
    }
    if constexpr (D == 128) {
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (j < 2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
    }
  };
  for (int t = tb; t < nt; t += NS) {
    step(t, std::integral_constant<int, 0>{});
    if (t + 1 < nt) step(t + 1, std::integral_constant<int, 1>{});
    if constexpr (NS > 2) if (t + 2 < nt) step(t + 2, std::integral_constant<int, 2>{});
    if constexpr (NS > 3) if (t + 3 < nt) step(t + 3, std::integral_constant<int, 3>{});
  }

  wait_vm_n<0>();  // no LDS-DMA may land after the work-group ends
  sage_finish<NW, D>(acc, m, l, part, su, sp, wave, lane, row, p, va + kvh * D, head, o);
}

// ---------------- software-pipelined main kernel ----------------
//
// Same work-group shape, unit/split mapping, LDS tile layouts and arithmetic as
// sage_attn_gen<128>, but each wave overlaps its own matrix and vector work: in the
// iteration of tile t it runs the online softmax of S(t) while it issues the score
// MFMAs of S(t+1) and the P(t-1) V(t-1) MFMAs, and it ends with the row max of S(t+1)
// and the LDS operands of iteration t+1 already in registers. The whole tile loop is
// one inline-assembly statement (sage_tile.inc; gen_sage_tile.py states the schedule,
// the register map and the hazards it respects); this function sets up its registers
// and LDS and finishes the output.
//
// LDS: K tiles in a ring of four 8 KB slots (tile j in slot j % 4), V^T tiles in
// another, and a table of 16 bytes per tile (liveness bits of its 64 keys, K scale).
// K(j) is read in iterations j-2 and j-1, V(j) in iterations j and j+1. Iteration t
// DMAs K(t+4) and V(t+2) into the slots of K(t) and V(t-2), last read in iteration
// t-1 (before the barrier at the top of iteration t); its DMA ops are waited for at
// the top of iteration t+2, before the first read of their tiles.
//
// Accumulator frames: before block A of iteration t the output accumulator holds
// P(..t-2) V in the frame of m(t-1); A and B add P(t-1) V(t-1), and the rescale by
// alpha(t) = 2^(m(t-1) - m(t)) follows B. The row sum l is rescaled before B, which
// adds this tile's sum (per wave half: the halves are combined once, at the end).
constexpr int kPipeMaxTiles = 512;  // tile table entries (8 KB of LDS): Skv <= 32768
constexpr int kPipeWaves = 4;       // 128 queries per work-group, two work-groups per CU

// QF: the kernel quantizes its own queries from bf16 q (qb; qi and qs are not read):
// each 16-row group of a wave is quantized exactly as prep_stats_q<D, -1, 16> does it
// (abs-max over the group's rows and channels, 127 / amax, rint), so the result equals
// the prologue-quantized path bit for bit, and the prologue skips Q (its bf16 read and
// int8 write). The queries of a unit are read by its work-groups before any of them
// writes the unit's output, so o may still alias q.
template <bool QF>
__global__ void __launch_bounds__(256, 2)
sage_attn_pipe(const int8_t* __restrict__ qi, const int8_t* __restrict__ ki, const uint8_t* __restrict__ vt_g,
               const float* __restrict__ qs, const u32x4* __restrict__ tab_g, const float* __restrict__ va,
               uint16_t* o, mx_attn_params p, int64_t sq_pad, int64_t skv_pad, SageSplit sp,
               const uint16_t* qb, float qmult) {
  constexpr int NW = kPipeWaves, QT = NW * 32, D = kPipeD;
  MX_STAMP(0);
  __shared__ __align__(16) unsigned char kring[4 * KTILEB];
  __shared__ __align__(16) unsigned char vring[4 * VTILEB];
  __shared__ __align__(16) u32x4 table[kPipeMaxTiles + 1];
  __shared__ __align__(16) float vas[kPipeD];  // the head's V channel scales, for the epilogue
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 31, h = lane >> 5;
  const int ntq = (p.Sq + QT - 1) / QT;
  const int nkt = (p.Skv + KT - 1) / KT;
  int L, tb = 0, nt = nkt, su = 0, part = -1;
  if (int(blockIdx.x) < sp.full) {
    L = xcd_remap(blockIdx.x, sp.full);
  } else {  // split units, part-major, XCD-grouped (see sage_attn_gen)
    const int nsu = (int(gridDim.x) - sp.full) / sp.parts;
    const int j = xcd_remap(int(blockIdx.x) - sp.full, int(gridDim.x) - sp.full);
    part = j / nsu;
    su = j - part * nsu;
    L = sp.full + su;
    tb = int(int64_t(part) * nkt / sp.parts);
    nt = int(int64_t(part + 1) * nkt / sp.parts);
  }
  const int head = L / ntq, qtile = L % ntq;
  const int kvh = head / (p.Hq / p.Hkv);
  const int row = qtile * QT + wave * 32 + n;  // < sq_pad
  const int last = nt - 1;

  // K/V^T DMA of a tile: 8 K ops and 8 V^T ops of 1 KB, two of each per wave. K op j
  // (j = 2w, 2w+1) fills rows (j & 1) * 32 + lane / 2 of d-chunk w (16-byte halves
  // swapped on rows 32..63); V^T op j fills channel rows 16 j + lane / 4. A tile past the
  // last is replaced by the last.
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int kr = lane >> 1, vr = lane >> 2;
  const uint32_t lk0 = uint32_t(kr * D + ((lane & 1) << 4));
  const uint32_t lk1 = uint32_t((32 + kr) * D + (((lane & 1) ^ 1) << 4));
  const uint32_t lv = uint32_t(vr) * uint32_t(skv_pad) + uint32_t(((lane & 3) ^ ((vr >> 2) & 3)) << 4);
  const uint32_t ksoff = uint32_t(wave_u * 32), vsoff = uint32_t(2 * wave_u * 16) * uint32_t(skv_pad);
  const uint32_t vstep = uint32_t(16) * uint32_t(skv_pad);
  const __amdgpu_buffer_rsrc_t rk_r = buf_rsrc(ki + int64_t(kvh) * skv_pad * D, uint32_t(skv_pad * D));
  const __amdgpu_buffer_rsrc_t rv_r = buf_rsrc(vt_g + int64_t(kvh) * D * skv_pad, uint32_t(skv_pad * D));
  auto dma_k = [&](int tile, int slot) __attribute__((always_inline)) {
    const uint32_t so = ksoff + uint32_t((tile < last ? tile : last) * (KT * D));
    unsigned char* d = kring + (slot & 3) * KTILEB + 2 * wave_u * 1024;
    buf2lds16(rk_r, lk0, so, (MXA_LDS void*)d);
    buf2lds16(rk_r, lk1, so, (MXA_LDS void*)(d + 1024));
  };
  auto dma_v = [&](int tile, int slot) __attribute__((always_inline)) {
    const uint32_t so = vsoff + uint32_t((tile < last ? tile : last) * KT);
    unsigned char* d = vring + (slot & 3) * VTILEB + 2 * wave_u * 1024;
    buf2lds16(rv_r, lv, so, (MXA_LDS void*)d);
    buf2lds16(rv_r, lv, so + vstep, (MXA_LDS void*)(d + 1024));
  };
  // QF: this lane's 64 bf16 channels of its row (h * 16 + cc * 32 + [0, 16); rows past
  // Sq are 0), loaded before the tile DMA so the quantization below waits for them only
  // (unconditional loads of a clamped row, zeroed afterwards: no per-lane branches)
  u32x4 raw[8];
  if constexpr (QF) {
    const int rc = row < p.Sq ? row : p.Sq - 1;
    const uint16_t* src = qb + int64_t(rc) * p.q_stride + int64_t(head) * D + h * 16;
#pragma unroll
    for (int j = 0; j < 8; ++j) raw[j] = *reinterpret_cast<const u32x4*>(src + (j >> 1) * 32 + (j & 1) * 8);
  }
  dma_k(tb, tb);
  dma_k(tb + 1, tb + 1);
  dma_k(tb + 2, tb + 2);
  dma_k(tb + 3, tb + 3);
  dma_v(tb, tb);
  dma_v(tb + 1, tb + 1);
  dma_v(tb, tb + 3);  // stands in for V(tb - 1) (read with P(tb - 1) = 0): finite bytes

  i32x4 qf[4];
  float qscale;
  if constexpr (!QF) {
    const int8_t* src = qi + (int64_t(head) * sq_pad + row) * D + h * 16;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) qf[cc] = *reinterpret_cast<const i32x4*>(src + cc * 32);
    qscale = qs[int64_t(head) * (sq_pad / 16) + row / 16];
  } else {
    float x[8][8], am = 0.f;
    const uint32_t keep = row < p.Sq ? ~0u : 0u;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[j][e] = bf2f(uint16_t((raw[j][e >> 1] & keep) >> ((e & 1) * 16)));
        am = fmaxf(am, fabsf(x[j][e]));
      }
    // the 16-row group of this lane: lanes with the same n >> 4 in both wave halves
    // (DPP row rotations within each 16-lane row: no LDS round trips)
    am = fmaxf(am, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(am), 0x128, 0xf, 0xf, false)));
    am = fmaxf(am, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(am), 0x124, 0xf, 0xf, false)));
    am = fmaxf(am, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(am), 0x122, 0xf, 0xf, false)));
    am = fmaxf(am, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(am), 0x121, 0xf, 0xf, false)));
    am = fmaxf(am, other_half(am));
    const float inv = am > 0.f ? 127.f / am : 0.f;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const u32x2 lo = quant8(x[2 * cc], inv), hi = quant8(x[2 * cc + 1], inv);
      qf[cc] = i32x4{int(lo[0]), int(lo[1]), int(hi[0]), int(hi[1])};
    }
    qscale = am / 127.f * qmult;
  }
  // tile table (liveness bits, K scale; written by the prologue's prep_kv_quant): one
  // coalesced 16-byte load per lane; the entry past the last tile is read by the last
  // iteration (its result is unused)
  {
    const u32x4* tg = tab_g + int64_t(kvh) * (skv_pad / KT + 1);
    u32x4 e[(kPipeMaxTiles + NW * 64 - 1) / (NW * 64)];
#pragma unroll
    for (int j = 0; j < int(sizeof(e) / sizeof(e[0])); ++j) {
      const int i = int(threadIdx.x) + j * NW * 64;
      if (i < nkt) e[j] = tg[i];
    }
#pragma unroll
    for (int j = 0; j < int(sizeof(e) / sizeof(e[0])); ++j) {
      const int i = int(threadIdx.x) + j * NW * 64;
      if (i < nkt) table[i] = e[j];
    }
    if (threadIdx.x == 0) table[nkt] = u32x4{~0u, ~0u, 0u, 0u};
    if (threadIdx.x < D) vas[threadIdx.x] = va[kvh * D + threadIdx.x];
  }
  wait_vm_n<0>();
  __syncthreads();  // K(tb..tb+3), V(tb), V(tb+1) and the tile table are visible
  MX_STAMP(1);

  // per-lane LDS read bases
  const int krow = kperm(0, n);
  const uint32_t kbase = uint32_t(krow * 32 + ((h ^ ((krow >> 5) & 1)) << 4));
  const int vsw = (n >> 2) & 3;
  const uint32_t vbase0 = uint32_t(n * 64 + (((2 * h) ^ vsw) << 4));
  const uint32_t vbase1 = uint32_t(n * 64 + (((2 * h + 1) ^ vsw) << 4));
  const uint32_t kring_l = uint32_t(uintptr_t((MXA_LDS unsigned char*)kring));
  const uint32_t vring_l = uint32_t(uintptr_t((MXA_LDS unsigned char*)vring));
  const uint32_t table_l = uint32_t(uintptr_t((MXA_LDS u32x4*)table));

  // S(tb) (masked) and its row max; the first iteration's operand registers
  i32x16 s0, s1;
  {
    const unsigned char* kd = kring + (tb & 3) * KTILEB + kbase;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const i32x4 a0 = *reinterpret_cast<const i32x4*>(kd + cc * 2048);
      const i32x4 a1 = *reinterpret_cast<const i32x4*>(kd + cc * 2048 + 512);
      s0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, qf[cc], cc == 0 ? kScoreBias16 : s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, qf[cc], cc == 0 ? kScoreBias16 : s1, 0, 0, 0);
    }
  }
  const u32x4 tab0 = table[tb];
  const uint32_t lw0 = h ? tab0[1] : tab0[0];
  int im;
  {
    int mx = kDead;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (!((lw0 >> i) & 1u)) s0[i] = kDead;
      if (!((lw0 >> (16 + i)) & 1u)) s1[i] = kDead;
      mx = max(mx, max(s0[i], s1[i]));
    }
    im = max(mx, other_half_i(mx));
  }
  const i32x32 stb = __builtin_shufflevector(s0, s1, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17,
                                             18, 19, 20, 21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 31);
  i32x32 sbuf0 = stb, sbuf1 = stb;  // S(tb) goes to buffer tb % 2 (the other one is overwritten)
  i32x8 kt;                          // K(tb+1) chunk 0 of both key blocks
  i32x16 vtr;                        // V(tb) channel blocks 0, 1 (stands in for V(tb - 1))
  {
    const unsigned char* kd = kring + ((tb + 1) & 3) * KTILEB + kbase;
    const i32x4 k0 = *reinterpret_cast<const i32x4*>(kd), k1 = *reinterpret_cast<const i32x4*>(kd + 512);
    kt = __builtin_shufflevector(k0, k1, 0, 1, 2, 3, 4, 5, 6, 7);
    const unsigned char* vd = vring + (tb & 3) * VTILEB;
    const i32x4 a = *reinterpret_cast<const i32x4*>(vd + vbase0), b = *reinterpret_cast<const i32x4*>(vd + vbase1);
    const i32x4 c = *reinterpret_cast<const i32x4*>(vd + vbase0 + 2048);
    const i32x4 d = *reinterpret_cast<const i32x4*>(vd + vbase1 + 2048);
    vtr = __builtin_shufflevector(__builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7),
                                  __builtin_shufflevector(c, d, 0, 1, 2, 3, 4, 5, 6, 7), 0, 1, 2, 3, 4, 5, 6, 7, 8, 9,
                                  10, 11, 12, 13, 14, 15);
  }
  const i32x16 q16 = __builtin_shufflevector(__builtin_shufflevector(qf[0], qf[1], 0, 1, 2, 3, 4, 5, 6, 7),
                                             __builtin_shufflevector(qf[2], qf[3], 0, 1, 2, 3, 4, 5, 6, 7), 0, 1,
                                             2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
  const i32x16 bias = kScoreBias16;
  // table entries by tile parity (v[228:230] / v[232:234]), v231 = the second K op's
  // per-lane offset; the entry of tile tb goes to both parities
  const i32x4 tabi = __builtin_bit_cast(i32x4, tab0);
  i32x8 tabs = __builtin_shufflevector(tabi, tabi, 0, 1, 2, 3, 4, 5, 6, 7);
  tabs[3] = int(lk1);
  tabs[7] = int(lv + vstep);  // the second V^T op's per-lane offset
  i32x16 pbuf = {};  // P buffers; P(tb - 1) = 0
  f32x16 acc0 = {}, acc1 = {}, acc2 = {}, acc3 = {};
  // running max, exponent offset and scale of tile tb (the loop computes them for the
  // next tile at the end of each iteration): m = tmax unless every key is dead
  const float sc = fmaxf(qscale * fabsf(__uint_as_float(tab0[2])), 1e-30f), c2 = 12582912.f * sc;
  float m = __builtin_fmaf(__int_as_float(im), sc, -c2);  // -inf when every key of tile tb is dead
  float nm = (kLog2_448 - kSageHeadroom - fmaxf(m, -3.0e38f)) - c2;
  float l = 0.f, alpha0 = 1.f, alpha1 = 1.f;
  uint64_t pend0 = 0, pend1 = 0;  // the accumulators need no rescale at tile tb
  int t = tb;
  int s_0, s_1, s_2, m0save;  // scalar scratch of the loop (M0 is saved and restored)
  const uint32_t kdm0 = kring_l + uint32_t(2 * wave_u * 1024), vdm0 = vring_l + uint32_t(2 * wave_u * 1024);
  // scalar state of the loop: the LDS address of tile t+1's table entry, the buffer
  // offsets of K(t+4) and V^T(t+2) (this wave's ops), and the variant limits (tiles up
  // to klim - 1 DMA K(t+4) and V(t+2), up to vlim - 1 only V(t+2))
  uint32_t tabp = table_l + uint32_t(tb + 1) * 16u;
  uint32_t kso = ksoff + uint32_t(tb + 4) * uint32_t(KT * D), vso = vsoff + uint32_t(tb + 2) * uint32_t(KT);
  const int klim = last - 3, vlim = last - 1;
  const uint64_t hmask = 0xffffffff00000000ull;
  float sc_v = sc;
  const uint32_t kb_l = kring_l + kbase, vb0_l = vring_l + vbase0, vb1_l = vring_l + vbase1;
  // the buffer resources as plain words (gfx9 dword3: 32-bit data, no swizzle)
  auto rsrc_words = [](const void* base, uint32_t bytes) __attribute__((always_inline)) {
    const uint64_t a = uint64_t(uintptr_t(base));
    return i32x4{int(uint32_t(a)), int(uint32_t(a >> 32) & 0xffffu), int(bytes), 0x00020000};
  };
  const i32x4 rk = rsrc_words(ki + int64_t(kvh) * skv_pad * D, uint32_t(skv_pad * D));
  const i32x4 rv = rsrc_words(vt_g + int64_t(kvh) * D * skv_pad, uint32_t(skv_pad * D));
  asm volatile(SAGE_TILE_LOOP
               : "+{v[0:15]}"(acc0), "+{v[16:31]}"(acc1), "+{v[32:47]}"(acc2), "+{v[48:63]}"(acc3),
                 "+{v[64:95]}"(sbuf0), "+{v[96:127]}"(sbuf1), "+{v[128:143]}"(pbuf), "+{v[144:151]}"(kt),
                 "+{v[152:167]}"(vtr), "+{v219}"(m), "+{v220}"(l), "+{v226}"(im), "+{v[228:235]}"(tabs),
                 "+{v222}"(sc_v), "+{v223}"(nm), "+{v239}"(alpha0), "+{v225}"(alpha1), [t] "+s"(t),
                 [s0] "=&s"(s_0), [s1] "=&s"(s_1), [s2] "=&s"(s_2), [pend0] "+s"(pend0), [pend1] "+s"(pend1),
                 [m0save] "=&s"(m0save), [tabp] "+s"(tabp), [kso] "+s"(kso), [vso] "+s"(vso)
               : "{v[168:183]}"(q16), "{v[184:199]}"(bias), "{v216}"(kb_l), "{v217}"(vb0_l), "{v218}"(vb1_l),
                 "{v221}"(qscale), "{v236}"(lk0), "{v237}"(lv), [nt] "s"(nt), [klim] "s"(klim), [vlim] "s"(vlim),
                 [kdm0] "s"(kdm0), [vdm0] "s"(vdm0), [rk] "s"(rk), [rv] "s"(rv), [hmask] "s"(hmask),
                 [kdead] "s"(kDead)
               : "v200", "v201", "v202", "v203", "v204", "v205", "v206", "v207", "v208", "v209", "v210", "v211",
                 "v212", "v213", "v214", "v215", "v224", "v227", "v238", "vcc", "scc", "memory");
  wait_vm_n<0>();  // no LDS-DMA may land after the work-group ends
  MX_STAMP(2);
  f32x16 acc[4] = {acc0, acc1, acc2, acc3};
  l += other_half(l);  // the wave halves summed different keys of the same rows
  sage_finish<NW, D>(acc, m, l, part, su, sp, wave, lane, row, p, vas, head, o, kring);
#ifdef MX_STAMPS
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  MX_STAMP(3);
  if (threadIdx.x == 0) g_stamps[size_t(blockIdx.x) * 8 + 5] = uint64_t(part + 1);
#endif
}

}  // namespace

// Workspace carve-up (kept in one place for the host code and the kernels).
// Two main kernels: sage_attn_pipe (4 waves, 128 queries per work-group, two
// work-groups per CU; D = 128, key tiles up to kPipeMaxTiles) and sage_attn_gen (8
// waves, 256 queries, one work-group per CU; D = 64 or 128, any length). The choice
// depends on D and Skv only.
struct SageShape {
  bool pipe;
  int qt, nw, per_cu;
};
SageShape sage_shape(const mx_attn_params& p) {
  const bool pipe = p.D == kPipeD && (p.Skv + KT - 1) / KT <= kPipeMaxTiles;
  return pipe ? SageShape{true, kPipeWaves * 32, kPipeWaves, 2} : SageShape{false, 256, 8, 1};
}

// Work split of the attention grid. A grid of U units (head, query tile) on C
// work-group slots runs in ceil(U / C) rounds, and the last one leaves slots idle when
// C does not divide U (config 2 on the 8-wave kernel: 408 units on 256 CUs, 1.59
// rounds of work in 2). The last U % C units are therefore split by key range into S
// parts, S chosen to minimise the tail's length ceil(r S / C) / S in units; each part
// writes its unnormalised output and the last part to finish merges them.
// C is the nominal slot count of an MI355X (256 CUs times the work-groups per CU), not
// the current device's: the workspace size and layout are a pure function of the
// shape, and on a device with another CU count the split stays correct (only its
// balance changes).
constexpr int kNominalCUs = 256;
struct SagePlan {
  int full;   // work-groups that run a whole unit (a multiple of C, or all units)
  int units;  // split units (the last `units` units of the grid)
  int parts;  // parts per split unit
};
SagePlan sage_plan(const mx_attn_params& p) {
  const SageShape sh = sage_shape(p);
  const int64_t ntq = (int64_t(p.Sq) + sh.qt - 1) / sh.qt, U64 = ntq * p.Hq;
  const int nt = (p.Skv + kKvPad - 1) / kKvPad;
  const int C = kNominalCUs * sh.per_cu;
  SagePlan pl{int(U64 < 0x7fffffff ? U64 : 0x7fffffff), 0, 1};
  if (U64 >= 0x7fffffff) return pl;
  const int U = int(U64), r = U % C;
  if (r == 0) return pl;
  if (sh.per_cu == 2 && U <= C) {
    // The whole grid is one dispatch round: estimate the call's time for each part
    // count S (parts of >= 4 key tiles) from rates measured on an MI355X (D = 128 pipe
    // kernel, us): a work-group alone on its CU runs a 64-key tile in ~0.62, two
    // co-resident ones ~1.1 each; launch + set-up + finish ~7; a split adds its
    // partial stores and merge, ~4 + 0.75 S. Parts beyond the 512 slots run in further
    // rounds, each paying the set-up again. Unsplit wins wherever the parts would
    // only double up on CUs (e.g. 216 units of 17 tiles: 18 against 24 us split in
    // two); long units on few CUs still split (128 units of 32 tiles: 2 parts).
    double best = 0.0;
    for (int S = 1; S <= kMaxParts && (S == 1 || S * 4 <= nt); ++S) {
      const int64_t P = int64_t(U) * S;
      const double w = double(nt) / S;
      const int rounds = int((P + C - 1) / C);
      double t = 7.0 + (S > 1 ? 4.0 + 0.75 * S : 0.0);
      if (P <= kNominalCUs) t += w * 0.62;
      else t += rounds * w * 1.1 + (rounds - 1) * 7.0;
      if (S == 1 || t < best - 1e-9) best = t, pl.parts = S;
    }
    if (pl.parts > 1) pl.full = 0, pl.units = U;
  } else if (sh.per_cu == 1 && U <= C) {
    // The same for the 8-wave kernel (D = 64; one work-group per CU): ~1.0 us per tile,
    // ~3.5 us of set-up per round of parts, a split ~4.5 (measured: 192 units of 32
    // tiles 39 us unsplit against 44 in four parts; 120 units of 17 tiles 21 in two
    // parts against 23 unsplit)
    double best = 0.0;
    for (int S = 1; S <= kMaxParts && (S == 1 || S * 4 <= nt); ++S) {
      const int rounds = int((int64_t(U) * S + C - 1) / C);
      const double t = 7.0 + (S > 1 ? 4.5 : 0.0) + rounds * (double(nt) / S + 3.5);
      if (S == 1 || t < best - 1e-9) best = t, pl.parts = S;
    }
    if (pl.parts > 1) pl.full = 0, pl.units = U;
  } else {
    // Several rounds: split the last round's r units into S parts, S minimising the
    // round count of the parts per part, ceil(r S / C) / S
    double best = 1.0;
    for (int S = 2; S <= kMaxParts && S * 4 <= nt; ++S) {  // parts of >= 4 key tiles
      const double cost = double((int64_t(r) * S + C - 1) / C) / S;
      if (cost < best - 1e-9) best = cost, pl.parts = S;
    }
    if (pl.parts > 1) pl.full = U - r, pl.units = r;
  }
#ifdef MX_STAMPS
  if (const char* e = getenv("MX_SAGE_PARTS")) {  // debug builds: force the part count
    const int S = atoi(e);
    pl = SagePlan{U, 0, 1};
    if (S > 1) pl = SagePlan{U - r, r, S};
  }
#endif
  return pl;
}

// Epoch of one fused-prologue call: a per-process counter from a random start, never 0
// (a zeroed workspace holds no set flag).
uint64_t next_epoch() {
  static std::atomic<uint64_t> ctr{[] {
    uint64_t x = uint64_t(std::chrono::steady_clock::now().time_since_epoch().count()) * 0x9E3779B97F4A7C15ull;
    try {  // no entropy source: the clock alone (a start value only needs to differ between processes)
      std::random_device rd;
      x ^= (uint64_t(rd()) << 32) ^ uint64_t(rd());
    } catch (...) {
    }
    return x;
  }()};
  uint64_t e;
  do e = ctr.fetch_add(1, std::memory_order_relaxed);
  while (e == 0);
  return e;
}

mx_sage_layout sage_layout(const mx_attn_params& p) {
  mx_sage_layout L{};
  const SagePlan pl = sage_plan(p);
  L.split_units = pl.units;
  L.split_parts = pl.parts;
  L.split_qt = sage_shape(p).qt;
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
  L.tab = take(16 * size_t(p.Hkv) * size_t(L.skv_pad / kKvPad + 1));
  L.split = take(sizeof(float) * split_floats(sage_shape(p).nw, p.D) * size_t(pl.units) * pl.parts);
  L.cnt = take(sizeof(int) * size_t(pl.units));
  L.flg = take(sizeof(uint64_t) * size_t(p.Hkv) * size_t(nb));
  L.total = off;
  return L;
}

// Prologue: preconditions checked by the caller (fp8_ok: D == 64 or 128, q/k/v 2-byte
// aligned with any token stride, skv_pad * D < 2^32 for the 32-bit buffer offsets; ws
// 256-byte aligned and large enough).
// nr: null for the plain prologue, else {Q norm/rope, K norm/rope} applied on the fly
// (D == 128 and nr128_supported, checked by the caller).
template <int D>
hipError_t sage_quantize_d(const uint16_t* q, const uint16_t* k, const uint16_t* v, const mx_attn_params& p,
                           char* ws, hipStream_t s, const NormRope* nr, int q_group, bool skip_q) {
  const mx_sage_layout L = sage_layout(p);
  const int nb = (p.Skv + kStatTok - 1) / kStatTok;
  float* part = reinterpret_cast<float*>(ws + L.part);
  float* km = reinterpret_cast<float*>(ws + L.km);
  float* va = reinterpret_cast<float*>(ws + L.va);
  const int64_t qgroups = int64_t(p.Hq) * (L.sq_pad / 16);
  // skip_q: the attention kernel quantizes Q itself (sage_attn_pipe<true>)
  const int64_t blocks1 = int64_t(p.Hkv) * nb + (skip_q ? 0 : (qgroups + 3) / 4);
  if (blocks1 > 0x7fffffff) return hipErrorInvalidValue;
  const float qmult = p.scale * kLog2e;
  const NormRope none{};
  const NormRope nq = nr ? nr[0] : none, nk = nr ? nr[1] : none;
  const int mode = nr ? nr128_mode(nq) : -1;
  // the Q work-groups hold four consecutive 16-row groups of one head (sq_pad is a
  // multiple of 64), i.e. one 64-row block, for the QG = 64 variant
  static_assert(kSqPad % 64 == 0, "Q padding must cover whole 64-row blocks");
  decltype(&prep_stats_q<D, -1, 16>) stats;
  decltype(&prep_kv_quant<D, -1>) kvq;
  if constexpr (D == 128) {
    stats = q_group == 64 ? prep_stats_q<D, -1, 64>
          : mode < 0 ? prep_stats_q<D, -1, 16> : mode == kRopeNone ? prep_stats_q<D, kRopeNone, 16>
          : mode == kRopeInterleaved ? prep_stats_q<D, kRopeInterleaved, 16> : prep_stats_q<D, kRopeHalf, 16>;
    kvq = mode < 0 ? prep_kv_quant<D, -1> : mode == kRopeNone ? prep_kv_quant<D, kRopeNone>
        : mode == kRopeInterleaved ? prep_kv_quant<D, kRopeInterleaved> : prep_kv_quant<D, kRopeHalf>;
  } else {
    if (mode >= 0) return hipErrorInvalidValue;  // the fused norm/rope prologue is D = 128 only
    stats = q_group == 64 ? prep_stats_q<D, -1, 64> : prep_stats_q<D, -1, 16>;
    kvq = prep_kv_quant<D, -1>;
  }
  // one-pass K/V prologue (prep_kv_fused) for the plain prologue outside stream capture
#ifdef MX_STAMPS
  const bool debug_old = std::getenv("MX_DEBUG_OLD_PROLOGUE") != nullptr;  // debug builds: A/B of the two paths
#else
  constexpr bool debug_old = false;
#endif
  if (mode < 0 && nb <= kFoldNb && !debug_old) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const hipError_t ce = hipStreamIsCapturing(s, &cap);
    if (ce != hipSuccess) return ce;
    if (cap == hipStreamCaptureStatusNone) {
      hipLaunchKernelGGL(prep_kv_fused<D>, dim3(unsigned(int64_t(p.Hkv) * nb)), dim3(512), 0, s, k, v, p, nb,
                         L.skv_pad, part, km, va, reinterpret_cast<int8_t*>(ws + L.ki),
                         reinterpret_cast<float*>(ws + L.ks), reinterpret_cast<uint8_t*>(ws + L.vt),
                         reinterpret_cast<u32x4*>(ws + L.tab), reinterpret_cast<int*>(ws + L.cnt), L.split_units,
                         reinterpret_cast<uint64_t*>(ws + L.flg), next_epoch(),
                         g_fused_wait_ticks.load(std::memory_order_relaxed));
      if (!skip_q && qgroups > 0)  // Q blocks only (no statistics blocks: nb = 0)
        hipLaunchKernelGGL(stats, dim3(unsigned((qgroups + 3) / 4)), dim3(256), 0, s, q, k, v, p, 0, qmult,
                           L.sq_pad, part, reinterpret_cast<int8_t*>(ws + L.qi), reinterpret_cast<float*>(ws + L.qs),
                           nq, nk);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL(stats, dim3(unsigned(blocks1)), dim3(256), 0, s, q, k, v, p, nb, qmult, L.sq_pad, part,
                     reinterpret_cast<int8_t*>(ws + L.qi), reinterpret_cast<float*>(ws + L.qs), nq, nk);
  // up to kFoldNb statistics partials per head (Skv <= 8192) the K/V quantizer sums
  // them itself (each work-group re-reads its head's partials from L2); beyond, that
  // re-reading would outweigh the separate prep_finalize launch
  const int fold = nb <= kFoldNb ? nb : 0;
  if (!fold)
    hipLaunchKernelGGL(prep_finalize<D>, dim3(p.Hkv), dim3(D), 0, s, p, nb, (const float*)part, km, va,
                       reinterpret_cast<int*>(ws + L.cnt), L.split_units);
  hipLaunchKernelGGL(kvq, dim3(unsigned(L.skv_pad / kKvPad), p.Hkv), dim3(256), 0, s, k, v, p, L.skv_pad, km, va,
                     reinterpret_cast<int8_t*>(ws + L.ki), reinterpret_cast<float*>(ws + L.ks),
                     reinterpret_cast<uint8_t*>(ws + L.vt), nk, fold, (const float*)part,
                     reinterpret_cast<int*>(ws + L.cnt), L.split_units, reinterpret_cast<u32x4*>(ws + L.tab));
  return hipGetLastError();
}

void set_prologue_wait_ticks(uint64_t ticks) { g_fused_wait_ticks.store(ticks, std::memory_order_relaxed); }

hipError_t launch_sage_quantize(const uint16_t* q, const uint16_t* k, const uint16_t* v, const mx_attn_params& p,
                                char* ws, hipStream_t s, const NormRope* nr, int q_group) {
  if (p.D == 128) return sage_quantize_d<128>(q, k, v, p, ws, s, nr, q_group, false);
  if (p.D == 64) return sage_quantize_d<64>(q, k, v, p, ws, s, nr, q_group, false);
  return hipErrorInvalidValue;
}

hipError_t sage_attend_impl(uint16_t* o, const mx_attn_params& p, const char* ws, hipStream_t s,
                            const uint16_t* qb) {
  static_assert(kSqPad % 256 == 0 && kSqPad % (kPipeWaves * 32) == 0, "Q padding must cover whole query tiles");
  const mx_sage_layout L = sage_layout(p);
  const SageShape sh = sage_shape(p);
  const int ntq = (p.Sq + sh.qt - 1) / sh.qt;
  const int64_t units = int64_t(ntq) * p.Hq;
  if (units > 0x7fffffff) return hipErrorInvalidValue;
  const SageSplit sp{int(units) - L.split_units, L.split_parts,
                     reinterpret_cast<float*>(const_cast<char*>(ws) + L.split),
                     reinterpret_cast<int*>(const_cast<char*>(ws) + L.cnt)};
  const int64_t blocks = int64_t(sp.full) + int64_t(L.split_units) * L.split_parts;
  const auto qi = reinterpret_cast<const int8_t*>(ws + L.qi);
  const auto ki = reinterpret_cast<const int8_t*>(ws + L.ki);
  const auto vt = reinterpret_cast<const uint8_t*>(ws + L.vt);
  const auto qs = reinterpret_cast<const float*>(ws + L.qs);
  const auto va = reinterpret_cast<const float*>(ws + L.va);
  const float qmult = p.scale * kLog2e;
  if (sh.pipe && qb)
    hipLaunchKernelGGL(sage_attn_pipe<true>, dim3(unsigned(blocks)), dim3(sh.nw * 64), 0, s, qi, ki, vt, qs,
                       reinterpret_cast<const u32x4*>(ws + L.tab), va, o, p, L.sq_pad, L.skv_pad, sp, qb, qmult);
  else if (sh.pipe)
    hipLaunchKernelGGL(sage_attn_pipe<false>, dim3(unsigned(blocks)), dim3(sh.nw * 64), 0, s, qi, ki, vt, qs,
                       reinterpret_cast<const u32x4*>(ws + L.tab), va, o, p, L.sq_pad, L.skv_pad, sp, qb, qmult);
  else if (p.D == 128)
    hipLaunchKernelGGL((sage_attn_gen<128, kSageStages>), dim3(unsigned(blocks)), dim3(sh.nw * 64), 0, s, qi, ki, vt,
                       qs, reinterpret_cast<const float*>(ws + L.ks), va, o, p, L.sq_pad, L.skv_pad, sp);
  else if (p.D == 64)
    hipLaunchKernelGGL((sage_attn_gen<64, kSageStages>), dim3(unsigned(blocks)), dim3(sh.nw * 64), 0, s, qi, ki, vt,
                       qs, reinterpret_cast<const float*>(ws + L.ks), va, o, p, L.sq_pad, L.skv_pad, sp);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_sage_attend(uint16_t* o, const mx_attn_params& p, const char* ws, hipStream_t s) {
  return sage_attend_impl(o, p, ws, s, nullptr);
}

// The whole quantized call (plain prologue, Q per 16 tokens): on the D = 128 pipe
// kernel the attention kernel quantizes Q itself and the prologue reads only K and V;
// otherwise the prologue quantizes Q into the workspace.
hipError_t launch_sage_fp8(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                           const mx_attn_params& p, char* ws, hipStream_t s) {
  const bool fuse_q = sage_shape(p).pipe;
  hipError_t e = p.D == 128 ? sage_quantize_d<128>(q, k, v, p, ws, s, nullptr, 16, fuse_q)
               : p.D == 64  ? sage_quantize_d<64>(q, k, v, p, ws, s, nullptr, 16, false)
                            : hipErrorInvalidValue;
  if (e != hipSuccess) return e;
  return sage_attend_impl(o, p, ws, s, fuse_q ? q : nullptr);
}

}  // namespace mxa

#ifdef MX_STAMPS
extern "C" int mx_debug_stamps_sage(void* dst, size_t bytes) {
  return int(hipMemcpyFromSymbol(dst, HIP_SYMBOL(mxa::g_stamps), bytes, 0, hipMemcpyDeviceToHost));
}
#endif

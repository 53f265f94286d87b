// BF16 flash-attention forward for gfx950 (CDNA4), D = 128, non-causal, with an
// optional key-padding mask. Reference behaviour: src/kernels/attention.cu:157-290
// (flash_kernel), :92-139 (online_softmax), :141-155 (store_output).
//
// Design (MI355X-first, not a translation of the reference's mma.sync tiling):
//  * Scores are computed transposed, S^T = K * Q^T, with v_mfma_f32_32x32x16_bf16:
//    A = K rows (from LDS), B = Q^T (resident in VGPRs for the whole kernel). In
//    the 32x32 C layout each lane holds ONE query (column lane%32) and 16 keys, so
//    the running max and sum are per-lane scalars; the only cross-lane step is one
//    v_permlane32_swap between the two wave halves.
//  * K rows are fed to the score MFMA in a permuted order (bits 2 and 3 of the
//    row index swapped) so each lane's 16 score registers are exactly the 8-key
//    runs the P*V MFMA wants as its B operand: P never leaves registers.
//  * O^T = V^T * P^T with the same MFMA; the V^T operand comes straight from the
//    row-major V tile with ds_read_b64_tr_b16 (gfx950 transposing LDS read).
//  * K and V tiles (64 keys) are double-buffered in LDS, filled by
//    global_load_lds_dwordx4 (16 B per lane, no VGPR staging) one tile ahead, in
//    bank-conflict-free layouts whose read addresses are one per-lane register
//    plus compile-time offsets (no per-chunk address registers). The buffers are
//    distinct LDS objects and the tile loop is unrolled twice, so the compiler can
//    prove an in-flight DMA never aliases the buffers being read and does not
//    wait for it; waits are explicit, counted vmcnt.
//  * Two work-group shapes (selected at build time, MXA_BF16_KIND):
//     W8 (default): 8 waves of 32 queries, two waves per SIMD; per tile
//        S -> softmax -> P*V, the other wave on the SIMD fills MFMA gaps.
//     W4S: 4 waves of 2x32 queries (blocks A, B), one wave per SIMD, the blocks
//        staggered half a tile so each MFMA phase has independent softmax work:
//        S_A(t) || softmax_B(t-1); P_B V(t-1) || softmax_A(t); S_B(t); P_A V(t).
//    Within a phase, sched_group_barrier keeps LDS operand reads a few MFMAs
//    ahead of use and spreads the VALU work between MFMAs.
//  * Work-groups are remapped so one head's query tiles share an XCD (and its L2).
#include <type_traits>

#include "attn_common.hpp"

#ifndef MXA_BF16_KIND
#define MXA_BF16_KIND 8
#endif
#ifndef MXA_KPF
#define MXA_KPF 3
#endif
#ifndef MXA_VPF
#define MXA_VPF 2
#endif
#ifndef MXA_SVALU
#define MXA_SVALU 12
#endif

namespace mxa {

namespace {

constexpr int D = 128;
constexpr int KT = 64;               // keys per tile
constexpr int TILEB = KT * D * 2;    // bytes per K (or V) tile

// LDS tile layouts (each 16 KB, filled by 16 DMA ops of 1 KB):
//  K: [8 d-chunks of 16][64 rows][2 halves of 8 channels]; the 16-byte half is
//     XOR'd with row bit 3 so the 16 rows one ds_read_b128 pass touches land on
//     16 distinct bank groups. A lane's read address is one per-lane base plus
//     compile-time offsets (d-chunk * 2048 + key block * 1024).
//  V: [4 d-blocks of 32][64 rows][64 B]; a ds_read_b64_tr_b16 touches 4 rows x
//     64 B = 256 contiguous bytes per 32 lanes, and its address is again one base
//     plus compile-time offsets.
constexpr int K_CHUNK = 2048, V_BLOCK = 4096;

// Score-row -> key permutation inside a 32-key block: swap bits 2 and 3.
__device__ __forceinline__ int perm32(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

// Per-lane constants.
struct Lane {
  int lane, n, h;
  int kbase;  // K read base within a tile
  int vbase;  // V^T transposing-read base within a tile
  float c;    // |scale| * log2(e)
  __device__ __forceinline__ Lane(float c_) : c(c_) {
    lane = threadIdx.x & 63;
    n = lane & 31;
    h = lane >> 5;
    const int krow = perm32(n);
    kbase = krow * 32 + ((h ^ ((krow >> 3) & 1)) << 4);
    // ds_read_b64_tr_b16: lane i of a 16-lane group reads 8 bytes of row (i>>2),
    // columns d0 + 4*(i&3); lane j of the group receives column d0+j of those rows.
    const int g16 = lane >> 4, i16 = lane & 15;
    vbase = ((g16 >> 1) * 8 + (i16 >> 2)) * 64 + ((g16 & 1) * 16 + (i16 & 3) * 4) * 2;
  }
};

// Per-wave state of one 32-query block.
struct QBlock {
  bf16x8 q[8];     // Q^T fragments (MFMA B operand), d-chunk cc: 16 channels
  f32x16 acc[4];   // O^T, 4 blocks of 32 channels
  f32x16 s[2];     // scores of the current tile, 2 blocks of 32 keys
  bf16x8 p[4];     // P^T (MFMA B operand), 4 chunks of 16 keys
  float m, l, alpha;
};

__device__ __forceinline__ void qblock_init(QBlock& X, const uint16_t* q, const mx_attn_params& p, int row0,
                                            int head, const Lane& ln, uint32_t qsign) {
  int row = row0 + ln.n;
  row = row < p.Sq ? row : p.Sq - 1;
  const uint16_t* src = q + int64_t(row) * p.q_stride + head * D + ln.h * 8;
#pragma unroll
  for (int cc = 0; cc < 8; ++cc) {
    u32x4 raw = *reinterpret_cast<const u32x4*>(src + cc * 16);
    raw ^= qsign;  // negative softmax scale: negate Q (exact) and use |scale|
    X.q[cc] = __builtin_bit_cast(bf16x8, raw);
  }
#pragma unroll
  for (int db = 0; db < 4; ++db) X.acc[db] = f32x16{};
  X.m = -__builtin_inff();
  X.l = 0.f;
  X.alpha = 1.f;
}

// DMA of one 64-key K or V tile: op j writes 1 KB (64 lanes x 16 B); a wave
// issues NLD ops, ops j = jj*NW + wave.
template <int NW, bool IS_V>
__device__ __forceinline__ void load_tile(const uint16_t* src, int t, unsigned char* dst, const mx_attn_params& p,
                                          int64_t kvbase, int wave, int lane) {
  constexpr int NLD = 16 / NW;
  const int key0 = t * KT;
#pragma unroll
  for (int jj = 0; jj < NLD; ++jj) {
    const int j = jj * NW + wave;
    int row, col;
    if constexpr (IS_V) {  // d-block j/4, rows (j%4)*16 + lane/4, 16-byte chunk lane%4
      row = (j & 3) * 16 + (lane >> 2);
      col = (j >> 2) * 32 + (lane & 3) * 8;
    } else {  // d-chunk j/2, rows (j%2)*32 + lane/2, stored half lane%2
      row = (j & 1) * 32 + (lane >> 1);
      col = (j >> 1) * 16 + (((lane & 1) ^ ((row >> 3) & 1)) << 3);
    }
    int key = key0 + row;
    key = key < p.Skv ? key : p.Skv - 1;
    g2lds16(src + int64_t(key) * p.kv_stride + kvbase + col, (MXA_LDS void*)(dst + j * 1024));
  }
}

// Liveness byte of one key per lane, always issued (from K itself when there is
// no mask) so every tile issues the same number of vector-memory ops per wave.
__device__ __forceinline__ void load_live(const mx_attn_params& p, const uint16_t* k, int key, int& in_range,
                                          int& byte) {
  in_range = key < p.Skv;
  const int kc = key < p.Skv ? key : p.Skv - 1;
  byte = p.kv_valid ? int(p.kv_valid[kc]) : int(reinterpret_cast<const uint8_t*>(k)[0] | 1);
}

// S^T = K Q^T for one tile (16 MFMA); the first MFMA of each key block takes a
// literal zero accumulator (no register initialisation).
__device__ __forceinline__ void scores(const unsigned char* kd, QBlock& X, const Lane& ln) {
#pragma unroll
  for (int cc = 0; cc < 8; ++cc)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(kd + ln.kbase + cc * K_CHUNK + kb * 1024);
      X.s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, X.q[cc], cc == 0 ? f32x16{} : X.s[kb], 0, 0, 0);
    }
}

// O^T += V^T P^T for one tile (16 MFMA).
// Key chunk outer, channel block inner: consecutive MFMAs accumulate into four
// different registers, so none waits on the previous one's result.
__device__ __forceinline__ void pv(const unsigned char* vd, QBlock& X, const Lane& ln) {
#pragma unroll
  for (int kc = 0; kc < 4; ++kc)
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const unsigned char* va = vd + ln.vbase + db * V_BLOCK + kc * 16 * 64;
      const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((MXA_LDS bf16x4*)(va));
      const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((MXA_LDS bf16x4*)(va + 4 * 64));
      const bf16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      X.acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, X.p[kc], X.acc[db], 0, 0, 0);
    }
}

// Dead keys (padding mask, tail) -> score -inf.
__device__ __forceinline__ void mask_scores(QBlock& X, uint64_t live, const Lane& ln) {
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = kb * 32 + (i >> 3) * 16 + ln.h * 8 + (i & 7);
      if (!((live >> key) & 1)) X.s[kb][i] = -__builtin_inff();
    }
}

// Branch-free online softmax (base 2) of one tile. X.m is the running max in
// log2 units (score * |scale| * log2 e). It only moves when the tile max exceeds
// it by more than kLazyMax: softmax is invariant to the subtracted constant, so
// a stale max changes nothing but rounding while P stays <= 2^kLazyMax, and the
// O rescale (alpha != 1) becomes rare instead of happening on most early tiles.
constexpr float kLazyMax = 8.f;
__device__ __forceinline__ void softmax(QBlock& X, const Lane& ln) {
  const float c = ln.c;
  float mx = X.s[0][0];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, X.s[kb][i]);
  mx = fmaxf(mx, other_half(mx)) * c;
  const float mnew = mx > X.m + kLazyMax ? mx : X.m;
  X.alpha = X.m == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(X.m - mnew);
  X.m = mnew;
  const float base = mnew == -__builtin_inff() ? 0.f : mnew;
  float rs = 0.f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(X.s[kb][i], c, -base));
      X.s[kb][i] = e;
      rs += e;
    }
  rs += other_half(rs);
  X.l = X.l * X.alpha + rs;
#pragma unroll
  for (int kc = 0; kc < 4; ++kc) {
    u32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = pack_bf16x2(X.s[kc >> 1][(kc & 1) * 8 + 2 * j], X.s[kc >> 1][(kc & 1) * 8 + 2 * j + 1]);
    X.p[kc] = __builtin_bit_cast(bf16x8, w);
  }
}

__device__ __forceinline__ void rescale(QBlock& X) {
  if (!__all(X.alpha == 1.f)) {
#pragma unroll
    for (int db = 0; db < 4; ++db) X.acc[db] *= X.alpha;
  }
}

// Scheduling recipes for one 16-MFMA phase: LDS operand reads kept a few MFMAs
// ahead of use, VALU instructions spread between consecutive MFMAs.
template <int VALU>
__device__ __forceinline__ void sched_k() {
  __builtin_amdgcn_sched_group_barrier(0x100, MXA_KPF, 0);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if constexpr (VALU > 0) __builtin_amdgcn_sched_group_barrier(0x002, VALU, 0);
    if (i < 16 - MXA_KPF) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
}
template <int VALU>
__device__ __forceinline__ void sched_v() {
  __builtin_amdgcn_sched_group_barrier(0x100, 2 * MXA_VPF, 0);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if constexpr (VALU > 0) __builtin_amdgcn_sched_group_barrier(0x002, VALU, 0);
    if (i < 16 - MXA_VPF) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
  }
}

__device__ __forceinline__ void store_block(const QBlock& X, uint16_t* o, const mx_attn_params& p, int row0,
                                            int head, const Lane& ln) {
  const int row = row0 + ln.n;
  if (row >= p.Sq) return;
  const float inv = X.l > 0.f ? 1.f / X.l : 0.f;
  uint16_t* dst = o + int64_t(row) * p.o_stride + head * D + ln.h * 4;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint32_t* d32 = reinterpret_cast<uint32_t*>(dst + db * 32 + g * 8);
      d32[0] = pack_bf16x2(X.acc[db][g * 4] * inv, X.acc[db][g * 4 + 1] * inv);
      d32[1] = pack_bf16x2(X.acc[db][g * 4 + 2] * inv, X.acc[db][g * 4 + 3] * inv);
    }
}

// ---------------- W8: 8 waves x 32 queries, two waves per SIMD ----------------
// NS-stage K/V ring: tile t lives in stage t % NS; at the top of tile t the
// loads of tile t + NS - 1 go into the stage tile t - 1 used. Each tile issues
// exactly OPS vector-memory ops per wave, so "tile t has landed" is a counted
// vmcnt((NS - 2) * OPS) that leaves the younger tiles in flight.
#ifndef MXA_NS
#define MXA_NS 2
#endif
template <int NS>
__global__ void __launch_bounds__(512, 1)
flash_bf16_d128_w8(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                   uint16_t* __restrict__ o, mx_attn_params p, float c, uint32_t qsign) {
  constexpr int NW = 8, QT = NW * 32, NLD = 16 / NW, OPS = 2 * NLD;
  static_assert(NS >= 2 && NS <= 4, "2..4 stages");
  __shared__ __align__(16) unsigned char st0[2 * TILEB];
  __shared__ __align__(16) unsigned char st1[2 * TILEB];
  __shared__ __align__(16) unsigned char st2[2 * TILEB];
  __shared__ __align__(16) unsigned char st3[2 * TILEB];
  auto stage = [&](auto i) __attribute__((always_inline)) -> unsigned char* {
    constexpr int I = decltype(i)::value % NS;
    if constexpr (I == 0) return st0;
    else if constexpr (I == 1) return st1;
    else if constexpr (I == 2) return st2;
    else return st3;
  };
  const Lane ln(c);
  const int wave = threadIdx.x >> 6;
  const int ntq = (p.Sq + QT - 1) / QT;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int head = L / ntq, qtile = L % ntq;
  const int kvh = head / (p.Hq / p.Hkv);
  const int q0 = qtile * QT + wave * 32;
  const int nt = (p.Skv + KT - 1) / KT;
  const int64_t kvbase = int64_t(kvh) * D;

  QBlock A;
  qblock_init(A, q, p, q0, head, ln, qsign);

  __shared__ uint64_t live_tiles[kMaxLiveTiles];
  auto issue = [&](int t, unsigned char* dst) __attribute__((always_inline)) {
    load_tile<NW, false>(k, t, dst, p, kvbase, wave, ln.lane);
    load_tile<NW, true>(v, t, dst + TILEB, p, kvbase, wave, ln.lane);
  };
  issue(0, stage(std::integral_constant<int, 0>{}));
  if constexpr (NS > 2) if (1 < nt) issue(1, stage(std::integral_constant<int, 1>{}));
  if constexpr (NS > 3) if (2 < nt) issue(2, stage(std::integral_constant<int, 2>{}));
  build_live<NW, KT>(live_tiles, p, nt, wave, ln.lane);
  __syncthreads();  // bitmaps visible (once, before the pipelined loop)

  auto step = [&](int t, auto i) __attribute__((always_inline)) {
    constexpr int I = decltype(i)::value;
    const unsigned char* kd = stage(i);
    const unsigned char* vd = kd + TILEB;
    // tile t has landed unless it is among the last NS-2 tiles (then wait for all)
    if (t + NS - 2 < nt) wait_vm_n<(NS - 2) * OPS>();
    else wait_vm_n<0>();
    block_sync();
    const uint64_t live = tile_live<KT>(live_tiles, p, t);
    if (t + NS - 1 < nt) issue(t + NS - 1, stage(std::integral_constant<int, I + NS - 1>{}));
    scores(kd, A, ln);
    sched_k<0>();
    if (live != ~0ull) mask_scores(A, live, ln);
    softmax(A, ln);
    rescale(A);
    pv(vd, A, ln);
    sched_v<0>();
  };
  for (int t = 0; t < nt; t += NS) {
    step(t, std::integral_constant<int, 0>{});
    if (t + 1 < nt) step(t + 1, std::integral_constant<int, 1>{});
    if constexpr (NS > 2) if (t + 2 < nt) step(t + 2, std::integral_constant<int, 2>{});
    if constexpr (NS > 3) if (t + 3 < nt) step(t + 3, std::integral_constant<int, 3>{});
  }
  store_block(A, o, p, q0, head, ln);
}

// ---------------- W4S: 4 waves x (2 x 32) queries, staggered blocks ----------------
__global__ void __launch_bounds__(256, 1)
flash_bf16_d128_w4s(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                    uint16_t* __restrict__ o, mx_attn_params p, float c, uint32_t qsign) {
  constexpr int NW = 4, QT = NW * 64, NLD = 16 / NW;
  constexpr int NK = NLD + 1;  // K group: K tile + one liveness byte
  __shared__ __align__(16) unsigned char kb0[TILEB];
  __shared__ __align__(16) unsigned char kb1[TILEB];
  __shared__ __align__(16) unsigned char vb0[TILEB];
  __shared__ __align__(16) unsigned char vb1[TILEB];
  const Lane ln(c);
  const int wave = threadIdx.x >> 6;
  const int ntq = (p.Sq + QT - 1) / QT;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int head = L / ntq, qtile = L % ntq;
  const int kvh = head / (p.Hq / p.Hkv);
  const int q0 = qtile * QT + wave * 64;
  const int nt = (p.Skv + KT - 1) / KT;
  const int64_t kvbase = int64_t(kvh) * D;

  QBlock A, B;
  qblock_init(A, q, p, q0, head, ln, qsign);
  qblock_init(B, q, p, q0 + 32, head, ln, qsign);

  // prologue: K(0) (+ liveness) then V(0) in flight
  load_tile<NW, false>(k, 0, kb0, p, kvbase, wave, ln.lane);
  int live_in, live_byte;
  load_live(p, k, ln.lane, live_in, live_byte);
  load_tile<NW, true>(v, 0, vb0, p, kvbase, wave, ln.lane);

  // Tile t: kcur = K(t), vcur = V(t), vprev = V(t-1); knext/vnext receive K(t+1)/V(t+1).
  auto step = [&](int t, const unsigned char* kcur, const unsigned char* vcur, const unsigned char* vprev,
                  unsigned char* knext, unsigned char* vnext, auto first) __attribute__((always_inline)) {
    constexpr bool FIRST = decltype(first)::value;
    // top: K(t) and its liveness bytes have landed (V(t) may still be in flight)
    wait_vm_n<NLD>();
    __syncthreads();
    const uint64_t live = __ballot(live_in && live_byte);
    if (t + 1 < nt) {
      load_tile<NW, false>(k, t + 1, knext, p, kvbase, wave, ln.lane);
      load_live(p, k, (t + 1) * KT + ln.lane, live_in, live_byte);
    }
    // P1: S_A(t) || softmax_B(t-1)
    scores(kcur, A, ln);
    if constexpr (!FIRST) {
      softmax(B, ln);
      sched_k<MXA_SVALU>();
      rescale(B);
    } else {
      sched_k<0>();
    }
    if (live != ~0ull) mask_scores(A, live, ln);
    // P2: P_B V(t-1) || softmax_A(t)
    if constexpr (!FIRST) pv(vprev, B, ln);
    softmax(A, ln);
    if constexpr (!FIRST) sched_v<MXA_SVALU>();
    // mid: everyone is done with V(t-1); V(t) has landed
    wait_vm_n<NK>();
    __syncthreads();
    if (t + 1 < nt) load_tile<NW, true>(v, t + 1, vnext, p, kvbase, wave, ln.lane);
    // P3: S_B(t), then the rescale of O_A
    scores(kcur, B, ln);
    sched_k<0>();
    rescale(A);
    if (live != ~0ull) mask_scores(B, live, ln);
    // P4: P_A V(t)
    pv(vcur, A, ln);
    sched_v<0>();
  };

  step(0, kb0, vb0, vb1, kb1, vb1, std::true_type{});
  for (int t = 1; t < nt; t += 2) {
    step(t, kb1, vb1, vb0, kb0, vb0, std::false_type{});
    if (t + 1 < nt) step(t + 1, kb0, vb0, vb1, kb1, vb1, std::false_type{});
  }
  // drain: softmax_B(nt-1), P_B V(nt-1)
  softmax(B, ln);
  rescale(B);
  pv((nt - 1) & 1 ? vb1 : vb0, B, ln);

  store_block(A, o, p, q0, head, ln);
  store_block(B, o, p, q0 + 32, head, ln);
}

}  // namespace

// Launch the fast path. Preconditions (checked by the caller): D == 128,
// non-causal, q/k/v 16-byte aligned with token strides % 8 == 0, o 4-byte
// aligned with o_stride % 2 == 0.
hipError_t launch_flash_bf16_d128(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                                  const mx_attn_params& p, hipStream_t s) {
  const float c = __builtin_fabsf(p.scale) * kLog2e;
  const uint32_t qsign = p.scale < 0.f ? 0x80008000u : 0u;
  constexpr int QT = 256;  // both shapes cover 256 queries per work-group
  const int ntq = (p.Sq + QT - 1) / QT;
  const int64_t blocks = int64_t(ntq) * p.Hq;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
#if MXA_BF16_KIND == 8
  hipLaunchKernelGGL(flash_bf16_d128_w8<MXA_NS>, dim3(unsigned(blocks)), dim3(512), 0, s, q, k, v, o, p, c, qsign);
#else
  hipLaunchKernelGGL(flash_bf16_d128_w4s, dim3(unsigned(blocks)), dim3(256), 0, s, q, k, v, o, p, c, qsign);
#endif
  return hipGetLastError();
}

}  // namespace mxa

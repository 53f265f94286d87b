// BF16 flash-attention forward for gfx950 (CDNA4), head dim D in {64, 72, 128},
// optional causal mask with query offset, optional key-padding mask, GQA. Reference behaviour: src/kernels/attention.cu:157-290
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
//    buffer_load_dwordx4 ... lds (16 B per lane, no VGPR staging) through a
//    per-tile buffer resource, in bank-conflict-free layouts whose read addresses
//    are one per-lane register plus compile-time offsets. The buffers are
//    distinct LDS objects and the tile loop is unrolled twice, so the compiler can
//    prove an in-flight DMA never aliases the buffers being read and does not
//    wait for it; waits are explicit, counted vmcnt. DMA ops are spread one per
//    four MFMAs (a burst of them stalls the issuing waves for hundreds of cycles).
//  * Work-group: 8 waves of 32 queries, two waves per SIMD, ping-pong: the two
//    waves of a SIMD run the same program one period apart, so one issues the
//    tile's MFMAs while the other runs the softmax (VALU); measured ~5% faster
//    than all waves in lockstep. Within an MFMA phase, sched_group_barrier keeps
//    LDS operand reads a few MFMAs ahead of use (kKPrefetch / kVPrefetch).
//  * Work-groups are remapped so one head's query tiles share an XCD (and its L2).
#include <atomic>
#include <mutex>
#include <type_traits>
#include <utility>

#include "attn_common.hpp"


namespace mxa {


namespace {

constexpr int KT = 64;               // keys per tile
constexpr int kKPrefetch = 3;        // K operand reads issued this many MFMAs ahead (scores)
constexpr int kVPrefetch = 2;        // V operand reads issued this many MFMAs ahead (P V)

// LDS tile layouts (16 KB each at D = 128, filled by DMA ops of 1 KB):
//  K: [D/16 d-chunks of 16][64 rows][2 halves of 8 channels]; the 16-byte half is
//     XOR'd with row bit 3 so the 16 rows one ds_read_b128 pass touches land on
//     16 distinct bank groups. A lane's read address is one per-lane base plus
//     compile-time offsets (d-chunk * 2048 + key block * 1024).
//  V: [D/32 d-blocks of 32][64 rows][64 B]; a ds_read_b64_tr_b16 touches 4 rows x
//     64 B = 256 contiguous bytes per 32 lanes, and its address is again one base
//     plus compile-time offsets.
constexpr int K_CHUNK = 2048, V_BLOCK = 4096;

// Per-tile work for head dimension DH. D = 72 runs as 80 in the score MFMA (the
// K and Q operands' channels 72..79 are zeroed in registers, whatever bytes follow
// the head in memory) and as 96 in P V (output channels 72..95 are computed from
// neighbouring bytes and never stored; each output channel depends only on its
// own V column).
template <int DH>
struct Dims {
  static constexpr int NC = (DH + 15) / 16;          // 16-channel chunks of S = K Q^T
  static constexpr int NB = (DH + 31) / 32;          // 32-channel blocks of O = P V
  static constexpr int KOPS = 2 * NC, VOPS = 4 * NB;  // 1 KB DMA ops per K / V tile
  static constexpr int KTB = NC * K_CHUNK, VTB = NB * V_BLOCK;
};

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
template <int DH>
struct QBlock {
  static constexpr int NC = Dims<DH>::NC, NB = Dims<DH>::NB;
  bf16x8 q[NC];    // Q^T fragments (MFMA B operand), d-chunk cc: 16 channels
  f32x16 acc[NB];  // O^T, blocks of 32 channels
  f32x16 s[2];     // scores of the current tile, 2 blocks of 32 keys
  bf16x8 p[4];     // P^T (MFMA B operand), 4 chunks of 16 keys
  float m, l, alpha;
};

template <int DH>
__device__ __forceinline__ void qblock_init(QBlock<DH>& X, const uint16_t* q, const mx_attn_params& p, int row0,
                                            int head, const Lane& ln, uint32_t qsign) {
  int row = row0 + ln.n;
  row = row < p.Sq ? row : p.Sq - 1;
  const uint16_t* src = q + int64_t(row) * p.q_stride + head * DH + ln.h * 8;
#pragma unroll
  for (int cc = 0; cc < X.NC; ++cc) {
    u32x4 raw = {0, 0, 0, 0};  // channels past DH (D = 72) stay zero
    if (DH % 16 == 0 || cc * 16 + ln.h * 8 < DH) raw = *reinterpret_cast<const u32x4*>(src + cc * 16);
    raw ^= qsign;  // negative softmax scale: negate Q (exact) and use |scale|
    X.q[cc] = __builtin_bit_cast(bf16x8, raw);
  }
#pragma unroll
  for (int db = 0; db < X.NB; ++db) X.acc[db] = f32x16{};
  X.m = -__builtin_inff();
  X.l = 0.f;
  X.alpha = 1.f;
}

// DMA of one 64-key K or V tile: op j writes 1 KB (64 lanes x 16 B) of the LDS
// layout above; a wave issues ops j = jj*NW + wave (< KOPS or VOPS). The global side is a
// per-tile buffer resource starting at key t*64 of this KV head: rows at or past
// Skv fall outside it and load as zeros (no clamping), the per-lane part is a
// loop-invariant byte offset and the per-op part is wave-uniform, so an op costs
// no vector ALU work. Requires Skv * kv_stride * 2 < 2^32 and a wave-uniform
// `wave`.
struct TileAddr {
  uint32_t lk, lv;  // per-lane byte offsets of this wave's K and V ops
};
template <int NW>
__device__ __forceinline__ TileAddr tile_addr(const mx_attn_params& p, int wave, int lane) {
  const uint32_t kvs = uint32_t(p.kv_stride);
  TileAddr a;
  // K op j = jj*NW + wave: row (j&1)*32 + lane/2 (j&1 == wave&1), 16-byte half
  // ((lane&1) ^ row bit 3) of d-chunk j/2
  const uint32_t krow = uint32_t((wave & 1) * 32 + (lane >> 1));
  a.lk = (krow * kvs + uint32_t(((lane & 1) ^ ((lane >> 4) & 1)) << 3)) * 2u;
  // V op j: row (j&3)*16 + lane/4 (j&3 == wave&3), 16-byte chunk lane&3 of d-block j/4
  const uint32_t vrow = uint32_t((wave & 3) * 16 + (lane >> 2));
  a.lv = (vrow * kvs + uint32_t((lane & 3) * 8)) * 2u;
  return a;
}
template <int NW, bool IS_V, int DH>
__device__ __forceinline__ void load_tile(const uint16_t* src, int t, unsigned char* dst, const mx_attn_params& p,
                                          int64_t kvbase, int wave, const TileAddr& ta) {
  constexpr int NOPS = IS_V ? Dims<DH>::VOPS : Dims<DH>::KOPS;
  constexpr int NLD = (NOPS + NW - 1) / NW;
  const int key0 = t * KT;
  const __amdgpu_buffer_rsrc_t r =
      buf_rsrc(src + kvbase + int64_t(key0) * p.kv_stride, uint32_t(p.Skv - key0) * uint32_t(p.kv_stride) * 2u);
  auto op = [&](auto jjc) __attribute__((always_inline)) {
    constexpr int jj = decltype(jjc)::value;
    if constexpr (NOPS % NW != 0)
      if (jj * NW + wave >= NOPS) return;  // wave-uniform
    MXA_LDS void* d = (MXA_LDS void*)(dst + (jj * NW + wave) * 1024);
    if constexpr (IS_V) {  // d-block j/4 = jj*(NW/4) + wave/4: 64 bytes each
      buf2lds16(r, ta.lv, uint32_t((jj * (NW / 4) + (NW == 8 ? (wave >> 2) : 0)) * 64), d);
    } else {  // d-chunk j/2 = jj*(NW/2) + wave/2: 32 bytes each
      buf2lds16(r, ta.lk, uint32_t((jj * (NW / 2) + (wave >> 1)) * 32), d);
    }
  };
  static_for<NLD>(op);
}

// S^T = K Q^T for one tile (2 * NC MFMA); the first MFMA of each key block takes a
// literal zero accumulator (no register initialisation).
template <int DH>
__device__ __forceinline__ void scores(const unsigned char* kd, QBlock<DH>& X, const Lane& ln) {
#pragma unroll
  for (int cc = 0; cc < X.NC; ++cc)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      bf16x8 a = *reinterpret_cast<const bf16x8*>(kd + ln.kbase + cc * K_CHUNK + kb * 1024);
      // D = 72: the last chunk's upper 8 channels hold whatever follows the head in
      // memory (possibly NaN padding); zero them so 0 * Q stays 0
      if (DH % 16 != 0 && cc == X.NC - 1 && ln.h) a = bf16x8{};
      X.s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, X.q[cc], cc == 0 ? f32x16{} : X.s[kb], 0, 0, 0);
    }
}

// O^T += V^T P^T for one tile (4 * NB MFMA).
// Key chunk outer, channel block inner: consecutive MFMAs accumulate into
// different registers, so none waits on the previous one's result.
template <int DH>
__device__ __forceinline__ void pv(const unsigned char* vd, QBlock<DH>& X, const Lane& ln) {
#pragma unroll
  for (int kc = 0; kc < 4; ++kc)
#pragma unroll
    for (int db = 0; db < X.NB; ++db) {
      const unsigned char* va = vd + ln.vbase + db * V_BLOCK + kc * 16 * 64;
      const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((MXA_LDS bf16x4*)(va));
      const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((MXA_LDS bf16x4*)(va + 4 * 64));
      const bf16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      X.acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, X.p[kc], X.acc[db], 0, 0, 0);
    }
}

// Dead keys (padding mask, tail) -> score -inf.
// Score i of key block kb is key kb*32 + (i>>3)*16 + 8h + (i&7): shift the bitmap
// by 8h once, then every test is a compile-time bit position (no per-lane masks).
// `rel` is the last key of the tile this lane's query may see (causal; >= 63 when
// every key is visible), so key index kk is kept iff kk <= rel.
template <bool CAUSAL, int DH>
__device__ __forceinline__ void mask_scores(QBlock<DH>& X, uint64_t live, int rel, const Lane& ln) {
  const uint64_t lv = live >> (ln.h * 8);
  const uint32_t lo = uint32_t(lv), hi = uint32_t(lv >> 32);
  const int relh = rel - ln.h * 8;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int bit = kb * 32 + (i >> 3) * 16 + (i & 7);
      const uint32_t w = bit < 32 ? lo : hi;
      if (!((w >> (bit & 31)) & 1u) || (CAUSAL && bit > relh)) X.s[kb][i] = -__builtin_inff();
    }
}

// Causal limit of one lane's query (row) for tile t: the last visible key index
// within the tile, clamped to [-1, 63] (reference: key j visible iff
// j <= q_offset + row, attention.cu:108).
__device__ __forceinline__ int causal_rel(const mx_attn_params& p, int row, int t) {
  const int64_t r = int64_t(p.q_offset) + row - int64_t(t) * KT;
  return r < -1 ? -1 : (r > KT - 1 ? KT - 1 : int(r));
}

// Key tiles one work-group of queries [qbeg, qbeg + QT) needs: all of them, or
// under the causal mask those up to key q_offset + min(qbeg + QT, Sq) - 1.
template <bool CAUSAL>
__device__ __forceinline__ int tiles_needed(const mx_attn_params& p, int qbeg, int QT) {
  const int nt = (p.Skv + KT - 1) / KT;
  if constexpr (!CAUSAL) return nt;
  const int64_t last = int64_t(p.q_offset) + (qbeg + QT < p.Sq ? qbeg + QT : p.Sq);  // exclusive
  if (last <= 0) return 0;
  const int64_t e = last < p.Skv ? last : p.Skv;
  return int((e + KT - 1) / KT);
}

// Branch-free online softmax (base 2) of one tile. X.m is the running max in
// log2 units (score * |scale| * log2 e). It only moves when the tile max exceeds
// it by more than kLazyMax: softmax is invariant to the subtracted constant, so
// a stale max changes nothing but rounding while P stays <= 2^kLazyMax, and the
// O rescale (alpha != 1) becomes rare instead of happening on most early tiles.
constexpr float kLazyMax = 8.f;
template <int DH>
__device__ __forceinline__ void softmax(QBlock<DH>& X, const Lane& ln) {
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

template <int DH>
__device__ __forceinline__ void rescale(QBlock<DH>& X) {
  if (!__all(X.alpha == 1.f)) {
#pragma unroll
    for (int db = 0; db < X.NB; ++db) X.acc[db] *= X.alpha;
  }
}

// Scheduling recipes for one MFMA phase of NMF MFMAs: LDS operand reads kept a
// few MFMAs ahead of use, and LD vector-memory (LDS-DMA) ops spread evenly
// between the MFMAs, so no wave issues a burst of DMA ops at once.
template <int NMF, int LD>
__device__ __forceinline__ void sched_k() {
  constexpr int PF = kKPrefetch < NMF ? kKPrefetch : NMF;
  __builtin_amdgcn_sched_group_barrier(0x100, PF, 0);
#pragma unroll
  for (int i = 0; i < NMF; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (LD && (i * LD) / NMF != ((i + 1) * LD) / NMF) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    if (i < NMF - PF) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
}
template <int NMF, int LD>
__device__ __forceinline__ void sched_v() {
  constexpr int PF = kVPrefetch < NMF ? kVPrefetch : NMF;
  __builtin_amdgcn_sched_group_barrier(0x100, 2 * PF, 0);
#pragma unroll
  for (int i = 0; i < NMF; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (LD && (i * LD) / NMF != ((i + 1) * LD) / NMF) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    if (i < NMF - PF) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
  }
}

template <int DH>
__device__ __forceinline__ void store_block(const QBlock<DH>& X, uint16_t* o, const mx_attn_params& p, int row0,
                                            int head, const Lane& ln) {
  const int row = row0 + ln.n;
  if (row >= p.Sq) return;
  const float inv = X.l > 0.f ? 1.f / X.l : 0.f;
  uint16_t* dst = o + int64_t(row) * p.o_stride + head * DH + ln.h * 4;
#pragma unroll
  for (int db = 0; db < X.NB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (DH % 32 != 0 && db * 32 + g * 8 >= DH) continue;  // D = 72: channels 72..95 are not output
      uint32_t* d32 = reinterpret_cast<uint32_t*>(dst + db * 32 + g * 8);
      d32[0] = pack_bf16x2(X.acc[db][g * 4] * inv, X.acc[db][g * 4 + 1] * inv);
      d32[1] = pack_bf16x2(X.acc[db][g * 4 + 2] * inv, X.acc[db][g * 4 + 3] * inv);
    }
}

// The same store through LDS (D = 64 / 128, o 16-byte aligned, o_stride % 8 == 0): the
// wave writes its 32 x DH output block into its own LDS region (16-byte chunks of row
// n XOR-swizzled by n), then every lane stores 16 contiguous bytes, so one store
// instruction writes 1 KB of whole rows instead of 4-byte pieces of 32 rows. The
// caller has passed a work-group barrier after the tile loop (the region is a K/V
// buffer).
template <int DH>
__device__ __forceinline__ void store_block_lds(const QBlock<DH>& X, uint16_t* o, const mx_attn_params& p,
                                                int row0, int head, const Lane& ln, unsigned char* wbuf) {
  static_assert(DH % 32 == 0, "whole 16-byte chunks per wave half");
  constexpr int CH = DH / 8, RB = DH * 2;
  const float inv = X.l > 0.f ? 1.f / X.l : 0.f;
#pragma unroll
  for (int db = 0; db < X.NB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int phys = (db * 4 + g) ^ (ln.n & (CH - 1));
      u32x2 w = {pack_bf16x2(X.acc[db][g * 4] * inv, X.acc[db][g * 4 + 1] * inv),
                 pack_bf16x2(X.acc[db][g * 4 + 2] * inv, X.acc[db][g * 4 + 3] * inv)};
      *reinterpret_cast<MXA_LDS u32x2*>((MXA_LDS unsigned char*)wbuf + ln.n * RB + phys * 16 + ln.h * 8) = w;
    }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
  for (int i = 0; i < 32 * CH / 64; ++i) {
    const int idx = i * 64 + ln.lane, r = idx / CH, c = idx % CH;
    const u32x4 val =
        *reinterpret_cast<const MXA_LDS u32x4*>((MXA_LDS unsigned char*)wbuf + r * RB + ((c ^ (r & (CH - 1))) * 16));
    const int row = row0 + r;
    if (row < p.Sq) *reinterpret_cast<u32x4*>(o + int64_t(row) * p.o_stride + head * DH + c * 8) = val;
  }
}

// ---------------- PP: 8 waves x 32 queries, ping-pong groups ----------------
// Waves w and w + 4 share a SIMD. Group A (waves 0-3) and group B (waves 4-7)
// run the same per-tile program offset by one period, so in every period one
// wave of each SIMD issues only MFMA (P(t) V(t), then S(t+1)) and the other only
// VALU (the online softmax); the SIMD keeps the matrix core busy with the first
// and fills the issue gaps with the second. Two work-group barriers per tile
// separate the periods:
//   period 2t+1: A: P V(t), S(t+1)    B: softmax(t)
//   period 2t+2: A: softmax(t+1)       B: P V(t), S(t+1)
// K(t+2) and V(t+1) go into the buffers of K(t) and V(t-1), both last read in
// period 2t; group A issues all of their DMA ops during its MFMA period 2t+1
// (8 per wave, one per four MFMAs), and waits for them at the top of tile t+1.
// Key-range split of the grid's last round (non-causal). The main launch runs the
// first `full` units (head, 256-query tile) whole; a second launch of the same kernel
// (SPLIT) runs each of the last `units` units as `parts` work-groups over consecutive
// key-tile ranges, and each writes its normalised partial output, scaled into fp16's
// range per query, with (m, l, scale) to a device region; bf16_split_merge combines
// the parts. Part-major work-group order: the work-groups of one XCD run one key range
// of consecutive units (mostly one head), so its L2 serves the K/V tiles they share.
struct BfSplit {
  uint16_t* po;  // [units][parts][256 queries][DH] fp16 partial outputs (o / scale)
  f32x4* ml;     // [units][parts][256 queries] {m (log2 units), l, scale, 0}
  int full, units, parts;
};

// Normalised partial of one 32-query block: o = acc / l, stored as fp16(o * 2^(15-e))
// with 2^(e-15) beside it, where e is the exponent of the query's largest |o| (so
// every stored value lies below 2^15 and keeps fp16's 11 significant bits relative
// to the row's largest). A query with no live key in the range stores l = 0.
template <int DH>
__device__ __forceinline__ void store_partial(const QBlock<DH>& X, const BfSplit& sp, int su, int part, int lrow,
                                              const Lane& ln) {
  float amax = 0.f;  // over the stored channels (D = 72: 72..95 hold padding products)
#pragma unroll
  for (int db = 0; db < X.NB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (DH % 32 == 0 || db * 32 + (i >> 2) * 8 < DH) amax = fmaxf(amax, __builtin_fabsf(X.acc[db][i]));
  amax = fmaxf(amax, other_half(amax));
  const float inv = X.l > 0.f ? 1.f / X.l : 0.f;
  int e = __builtin_amdgcn_frexp_expf(amax * inv);
  e = e < -100 ? -100 : (e > 140 ? 140 : e);
  const float sc = __builtin_ldexpf(inv, 15 - e);
  const size_t blk = size_t(su) * sp.parts + part;
  uint16_t* dst = sp.po + (blk * 256 + lrow) * DH + ln.h * 4;
#pragma unroll
  for (int db = 0; db < X.NB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (DH % 32 != 0 && db * 32 + g * 8 >= DH) continue;
      using h2 = __attribute__((ext_vector_type(2))) _Float16;
      const h2 a = __builtin_convertvector((f32x2){X.acc[db][g * 4] * sc, X.acc[db][g * 4 + 1] * sc}, h2);
      const h2 b = __builtin_convertvector((f32x2){X.acc[db][g * 4 + 2] * sc, X.acc[db][g * 4 + 3] * sc}, h2);
      u32x2 w = {__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)};
      *reinterpret_cast<u32x2*>(dst + db * 32 + g * 8) = w;
    }
  // both wave halves store the query's (identical) record: a branch on the half here
  // changes the compiler's schedule of the whole tile loop for the worse
  sp.ml[blk * 256 + lrow] = f32x4{X.m, X.l, __builtin_ldexpf(1.f, e - 15), 0.f};
}

// Occupancy: one work-group of 8 waves per CU, two waves per SIMD. The causal kernels
// state that target (waves_per_eu 2): aiming for three waves per SIMD, the compiler caps
// a kernel at 168 VGPRs, and the causal tile loop needs 177 (the per-lane diagonal
// mask), so it gave up the LDS operand prefetch (one operand register set, each read
// waited for before its MFMA; config-2 shape 176 -> 146 us with the target stated).
// The non-causal kernels keep the equivalent of __launch_bounds__(512, 1): the stated
// target changes their schedule for the worse at D = 64 and not at all at D = 128.

template <int DH, bool CAUSAL, bool SPLIT>
__global__ void __attribute__((amdgpu_flat_work_group_size(CAUSAL || DH == 128 ? 512 : 1, 512),
                               amdgpu_waves_per_eu(CAUSAL || DH == 128 ? 2 : 1, CAUSAL || DH == 128 ? 2 : 8)))
flash_bf16_pp(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
              uint16_t* __restrict__ o, mx_attn_params p, float c, uint32_t qsign, BfSplit sp) {
  using Dm = Dims<DH>;
  constexpr int NW = 8, QT = NW * 32;
  constexpr int LDK = (Dm::KOPS + 3) / 4, LDV = (Dm::VOPS + 3) / 4;  // loop DMA ops per group-A wave
  __shared__ __align__(16) unsigned char kb0[Dm::KTB];
  __shared__ __align__(16) unsigned char kb1[Dm::KTB];
  __shared__ __align__(16) unsigned char vb0[Dm::VTB];
  __shared__ __align__(16) unsigned char vb1[Dm::VTB];
  __shared__ uint64_t live_tiles[kMaxLiveTiles];
  MX_STAMP(0);
  const Lane ln(c);
  const int wave = threadIdx.x >> 6;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const bool group_a = wave < 4;
  const int ntq = (p.Sq + QT - 1) / QT;
  const int Lx = xcd_remap(blockIdx.x, gridDim.x);
  int L = Lx, su = 0, part = 0;
  if constexpr (SPLIT) {  // part-major: su = split unit, part = key range
    part = Lx / sp.units;
    su = Lx - part * sp.units;
    L = sp.full + su;
  }
  // causal: query tiles with the most key tiles first
  const int head = L / ntq, qtile = CAUSAL ? ntq - 1 - L % ntq : L % ntq;
  const int kvh = head / (p.Hq / p.Hkv);
  const int q0 = qtile * QT + wave * 32;
  const int ntk = tiles_needed<CAUSAL>(p, qtile * QT, QT);
  // key tiles [tb, nt) of this work-group
  const int tb = SPLIT ? int(int64_t(part) * ntk / sp.parts) : 0;
  const int nt = SPLIT ? int(int64_t(part + 1) * ntk / sp.parts) : ntk;
  const int64_t kvbase = int64_t(kvh) * DH;
  const TileAddr ta8 = tile_addr<8>(p, wave_u, ln.lane);      // prologue: all 8 waves load
  const TileAddr ta4 = tile_addr<4>(p, wave_u & 3, ln.lane);  // loop: group A loads

  QBlock<DH> A;
  if (CAUSAL && nt == 0) {  // causal: no visible key for any query of the work-group -> 0
    qblock_init(A, q, p, q0, head, ln, qsign);
    store_block(A, o, p, q0, head, ln);
    return;
  }
  // 16-byte aligned mask: its loads go first and are folded after the tile and Q loads
  const bool mask16 = p.kv_valid && (reinterpret_cast<uintptr_t>(p.kv_valid) & 15) == 0;
  Live16 lv16{};
  if (mask16) lv16 = live16_issue<NW>(p, nt, wave_u, ln.lane);
  load_tile<NW, false, DH>(k, tb, kb0, p, kvbase, wave_u, ta8);
  load_tile<NW, true, DH>(v, tb, vb0, p, kvbase, wave_u, ta8);
  if (nt > tb + 1) load_tile<NW, false, DH>(k, tb + 1, kb1, p, kvbase, wave_u, ta8);
  qblock_init(A, q, p, q0, head, ln, qsign);
  if (mask16) live16_finish<NW>(live_tiles, lv16, p, nt, wave_u, ln.lane);
  else build_live<NW, KT>(live_tiles, p, nt, wave, ln.lane);

  // MFMA period of tile t: P V(t) then S(t+1). S(t+1) on a stale buffer when
  // t + 1 == nt is harmless (never read). With LOAD, also the DMA of V(t+1) and
  // K(t+2) (clamped to the last tile so the ops are unconditional).
  auto mfma_part = [&](int t, const unsigned char* kc1, const unsigned char* vcur, unsigned char* kfree,
                       unsigned char* vfree, auto load) __attribute__((always_inline)) {
    __builtin_amdgcn_s_setprio(1);
    if constexpr (decltype(load)::value) {
      load_tile<4, true, DH>(v, t + 1 < nt ? t + 1 : nt - 1, vfree, p, kvbase, wave_u & 3, ta4);
      pv(vcur, A, ln);
      sched_v<4 * Dm::NB, LDV>();
      load_tile<4, false, DH>(k, t + 2 < nt ? t + 2 : nt - 1, kfree, p, kvbase, wave_u & 3, ta4);
      scores(kc1, A, ln);
      sched_k<2 * Dm::NC, LDK>();
    } else {
      pv(vcur, A, ln);
      sched_v<4 * Dm::NB, 0>();
      scores(kc1, A, ln);
      sched_k<2 * Dm::NC, 0>();
    }
    __builtin_amdgcn_s_setprio(0);
  };
  auto valu_part = [&](int t) __attribute__((always_inline)) {
    const uint64_t live = tile_live<KT>(live_tiles, p, t);
    const bool diag = CAUSAL && int64_t(p.q_offset) + q0 - int64_t(t) * KT < KT - 1;  // wave-uniform
    if (live != ~0ull || diag) mask_scores<CAUSAL>(A, live, diag ? causal_rel(p, q0 + ln.n, t) : KT - 1, ln);
    softmax(A, ln);
    rescale(A);
  };

  wait_vm_n<0>();
  __syncthreads();  // K(0), V(0), K(1) and the liveness bitmaps are visible
  MX_STAMP(1);
  if (group_a) {    // period -1: S_A(0)
    scores(kb0, A, ln);
    sched_k<2 * Dm::NC, 0>();
  }
  block_sync();
  if (group_a) {    // period 0: A softmax(tb), B S_B(tb)
    valu_part(tb);
  } else {
    scores(kb0, A, ln);
    sched_k<2 * Dm::NC, 0>();
  }

  // Tile t: kc1 = K(t+1), vcur = V(t); kfree / vfree receive K(t+2) / V(t+1).
  auto tile = [&](int t, const unsigned char* kc1, const unsigned char* vcur, unsigned char* kfree,
                  unsigned char* vfree) __attribute__((always_inline)) {
    wait_vm_n<0>();  // group A: K(t+1), V(t) landed
    block_sync();
    if (group_a) mfma_part(t, kc1, vcur, kfree, vfree, std::true_type{});
    else valu_part(t);
    block_sync();
    if (group_a) {
      if (t + 1 < nt) valu_part(t + 1);
    } else {
      mfma_part(t, kc1, vcur, kfree, vfree, std::false_type{});
    }
  };
  for (int t = tb; t < nt; t += 2) {
    tile(t, kb1, vb0, kb0, vb1);
    if (t + 1 < nt) tile(t + 1, kb0, vb1, kb1, vb0);
  }
  wait_vm_n<0>();  // no LDS-DMA may land after the work-group ends
  MX_STAMP(2);
  if constexpr (SPLIT) {
    store_partial(A, sp, su, part, wave * 32 + ln.n, ln);
  } else if constexpr (DH % 32 == 0) {
    if ((reinterpret_cast<uintptr_t>(o) & 15) == 0 && (p.o_stride & 7) == 0) {
      block_sync();  // every wave is done reading the K/V buffers
      const int wb = wave_u >> 1;
      unsigned char* buf = wb == 0 ? kb0 : wb == 1 ? kb1 : wb == 2 ? vb0 : vb1;
      store_block_lds(A, o, p, q0, head, ln, buf + (wave_u & 1) * 32 * DH * 2);
    } else {
      store_block(A, o, p, q0, head, ln);
    }
  } else {
    store_block(A, o, p, q0, head, ln);
  }
#ifdef MX_STAMPS
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  MX_STAMP(3);
#endif
}

// Merge of the split units' parts: one thread per (query, 8 channels). With
// M = max m_i and c_i = l_i 2^(m_i - M), o = sum c_i scale_i o_i / sum c_i (parts
// whose keys were all dead have l_i = 0 and drop out; no live key at all gives 0).
template <int DH>
__global__ void __launch_bounds__(256)
bf16_split_merge(uint16_t* __restrict__ o, mx_attn_params p, BfSplit sp) {
  constexpr int G = DH / 8, QT = 256;
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t rowg = idx / G;
  const int g = int(idx - rowg * G);
  if (rowg >= int64_t(sp.units) * QT) return;
  const int su = int(rowg / QT), lrow = int(rowg % QT);
  const int ntq = (p.Sq + QT - 1) / QT;
  const int L = sp.full + su, head = L / ntq, row = (L % ntq) * QT + lrow;
  if (row >= p.Sq) return;
  float M = -__builtin_inff();
  for (int i = 0; i < sp.parts; ++i) {
    const f32x4 t = sp.ml[(size_t(su) * sp.parts + i) * QT + lrow];
    if (t[1] > 0.f) M = fmaxf(M, t[0]);
  }
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, den = 0.f;
  for (int i = 0; i < sp.parts; ++i) {
    const size_t blk = (size_t(su) * sp.parts + i) * QT + lrow;
    const f32x4 t = sp.ml[blk];
    if (!(t[1] > 0.f)) continue;
    const float cw = t[1] * __builtin_amdgcn_exp2f(t[0] - M);
    den += cw;
    const float f = cw * t[2];
    using h8 = __attribute__((ext_vector_type(8))) _Float16;
    const h8 x = *reinterpret_cast<const h8*>(sp.po + blk * DH + g * 8);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += f * float(x[j]);
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  u32x4 w;
#pragma unroll
  for (int j = 0; j < 4; ++j) w[j] = pack_bf16x2(acc[2 * j] * inv, acc[2 * j + 1] * inv);
  uint32_t* d = reinterpret_cast<uint32_t*>(o + int64_t(row) * p.o_stride + int64_t(head) * DH + g * 8);
#pragma unroll
  for (int j = 0; j < 4; ++j) d[j] = w[j];
}

}  // namespace

namespace {

struct Bf16Plan {
  int full, units, parts;
};
constexpr int kBfMaxParts = 8;

// Split partials: ml [units][parts][256] {m, l, scale, 0} f32, then po
// [units][parts][256][D] fp16.
size_t bf16_split_bytes(int units, int parts, int D) {
  const size_t blocks = size_t(units) * parts * 256;
  return blocks * sizeof(f32x4) + (blocks * D * 2 + 255) / 256 * 256;
}

// The split partials live in this fixed region, one copy per device, held until the
// process ends: the library never allocates on the launch path. 16 MiB holds, at
// D = 128, 240 parts of 256 queries (e.g. 30 units x 8 parts, 48 x 5); the plan only
// considers splits that fit.
constexpr size_t kBfSplitBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char bf16_split_scratch[kBfSplitBytes];

// Split plan for a non-causal grid of U units on C CUs (one work-group per CU). The
// chip is power-limited: a CU runs a 64-key tile in ~1.29 us (D = 128) while at most
// ~165 CUs are busy, and the clock drops as more are (~2.0 us per tile with all 256
// busy; measured on MI355X). So the grid's last, partly filled round of r = U mod C
// units costs nearly as much as a full one only when r is small; for r near C its CUs
// run faster and splitting buys little. The estimate below compares that round with
// splitting its units into S key ranges: rounds of min(C, remaining parts) busy CUs,
// each part nt/S tiles plus ~2 tiles of fixed work (Q load, first tiles, partial
// store), then the merge (partial bytes at ~3 TB/s plus ~4 us) and ~3 us for the
// second launch when whole rounds precede it. S minimises the estimate; no split
// unless it wins by 5 %, and only splits whose partials fit the fixed region. Measured: U = 2..32 units 1.9-3.2x faster, config-2 shape
// (408 units, r = 152) and 120 units of 17 tiles unsplit.
Bf16Plan bf16_plan(const mx_attn_params& p, int C) {
  constexpr int QT = 256;
  const int64_t U64 = int64_t((p.Sq + QT - 1) / QT) * p.Hq;
  const int nt = (p.Skv + KT - 1) / KT;
  Bf16Plan pl{int(U64), 0, 1};
  if (p.causal || C <= 0 || U64 >= 0x7fffffff) return pl;
  const int U = int(U64), r = U % C;
  if (r == 0) return pl;
  const double t0 = 1.29e-6 * (0.4 + 0.6 * p.D / 128.0);  // s per tile per CU, <= kBusyFast busy CUs
  constexpr double kBusyFast = 165.0;
  auto tile_s = [&](int busy) { return t0 * (busy > kBusyFast ? busy / kBusyFast : 1.0); };
  const double whole = nt * tile_s(r);
  double best = 0.95 * whole;
  for (int S = 2; S <= kBfMaxParts && S * 4 <= nt; ++S) {
    if (bf16_split_bytes(r, S, p.D) > kBfSplitBytes) break;
    double cost = U > r ? 3e-6 : 0.0;
    for (int64_t left = int64_t(r) * S; left > 0; left -= C)
      cost += (double(nt) / S + 2.0) * tile_s(int(left < C ? left : C));
    cost += double(r) * S * QT * (2 * p.D + 16) / 3e12 + 4e-6;
    if (cost < best) best = cost, pl.parts = S;
  }
  if (pl.parts > 1) pl.full = U - r, pl.units = r;
  return pl;
}

// Per-device state of the split. cus is read without a lock (every thread that races
// to fill it stores the same value). The region's address and the ordering event are
// set up once per device, on the first call that splits; after that a split call
// takes the device's mutex only to order itself after the previous split call
// (stream wait on the event, launches, event record), so calls on different streams
// never share the region at the same time. Calls that do not split (the large grids,
// causal calls, calls under stream capture) take no lock and touch no shared state.
constexpr int kMaxDev = 64;
struct SplitDevice {
  std::atomic<int> cus{0};
  std::once_flag once;
  hipError_t setup = hipSuccess;
  void* region = nullptr;
  hipEvent_t done = nullptr;
  std::mutex mu;
};
SplitDevice g_split[kMaxDev];

int device_cus(SplitDevice& R, int dev) {
  int n = R.cus.load(std::memory_order_relaxed);
  if (n == 0 && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
    R.cus.store(n, std::memory_order_relaxed);
  return n;
}

hipError_t split_setup(SplitDevice& R) {
  std::call_once(R.once, [&R] {
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(bf16_split_scratch));
    if (e == hipSuccess && (!ptr || reinterpret_cast<uintptr_t>(ptr) % 256)) e = hipErrorInvalidValue;
    if (e == hipSuccess) e = hipEventCreateWithFlags(&R.done, hipEventDisableTiming);
    if (e == hipSuccess) R.region = ptr;
    R.setup = e;
  });
  return R.setup;
}

}  // namespace

int flash_bf16_split_plan(const mx_attn_params& p, int cus, int* full, int* units, int* parts) {
  const Bf16Plan pl = bf16_plan(p, cus);
  *full = pl.full, *units = pl.units, *parts = pl.parts;
  return 0;
}

// Launch the fast path. Preconditions (checked by the caller): D in {64, 72, 128},
// q/k/v/o 2-byte aligned, Skv * kv_stride * 2 < 2^32. No allocation, no host sync.
hipError_t launch_flash_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                             const mx_attn_params& p, hipStream_t s) {
  const float c = __builtin_fabsf(p.scale) * kLog2e;
  const uint32_t qsign = p.scale < 0.f ? 0x80008000u : 0u;
  constexpr int QT = 256;  // queries per work-group
  const int ntq = (p.Sq + QT - 1) / QT;
  const int64_t blocks = int64_t(ntq) * p.Hq;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  if (p.D != 128 && p.D != 64 && p.D != 72) return hipErrorInvalidValue;
  const bool cz = p.causal != 0;

  Bf16Plan pl{int(blocks), 0, 1};
  SplitDevice* R = nullptr;
  if (!cz) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev >= 0 && dev < kMaxDev) {
      R = &g_split[dev];
      pl = bf16_plan(p, device_cus(*R, dev));
    }
    if (pl.parts > 1) {
      // a captured graph may replay while eager calls use the region: capture runs unsplit
      hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(s, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone ||
          split_setup(*R) != hipSuccess)
        pl = Bf16Plan{int(blocks), 0, 1};
    }
  }

  BfSplit sp{nullptr, nullptr, pl.full, pl.units, pl.parts};
  auto run = [&](auto kern, int64_t n) {
    if (n > 0) hipLaunchKernelGGL(kern, dim3(unsigned(n)), dim3(512), 0, s, q, k, v, o, p, c, qsign, sp);
  };
  auto go = [&](auto DHc) -> hipError_t {
    constexpr int DH = decltype(DHc)::value;
    if (cz) {
      run(flash_bf16_pp<DH, true, false>, blocks);
      return hipGetLastError();
    }
    run(flash_bf16_pp<DH, false, false>, pl.full);
    if (pl.parts > 1) {
      std::lock_guard<std::mutex> lock(R->mu);
      hipError_t e2 = hipStreamWaitEvent(s, R->done, 0);
      if (e2 != hipSuccess) return e2;
      const size_t blocks_ml = size_t(pl.units) * pl.parts * 256;
      sp.ml = static_cast<f32x4*>(R->region);
      sp.po = reinterpret_cast<uint16_t*>(static_cast<char*>(R->region) + blocks_ml * sizeof(f32x4));
      run(flash_bf16_pp<DH, false, true>, int64_t(pl.units) * pl.parts);
      const int64_t threads = int64_t(pl.units) * QT * (DH / 8);
      hipLaunchKernelGGL(bf16_split_merge<DH>, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, s, o, p, sp);
      e2 = hipGetLastError();
      if (e2 != hipSuccess) return e2;
      return hipEventRecord(R->done, s);
    }
    return hipGetLastError();
  };
  switch (p.D) {
    case 128: return go(std::integral_constant<int, 128>{});
    case 64: return go(std::integral_constant<int, 64>{});
    default: return go(std::integral_constant<int, 72>{});
  }
}

}  // namespace mxa

#ifdef MX_STAMPS
extern "C" int mx_debug_stamps(void* dst, size_t bytes) {
  return int(hipMemcpyFromSymbol(dst, HIP_SYMBOL(mxa::g_stamps), bytes, 0, hipMemcpyDeviceToHost));
}
#endif

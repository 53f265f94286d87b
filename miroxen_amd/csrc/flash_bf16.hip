// BF16 flash-attention forward for gfx950 (CDNA4), D = 128, non-causal, with an
// optional key-padding mask. Reference behaviour: src/kernels/attention.cu:157-290
// (flash_kernel), :92-139 (online_softmax), :141-155 (store_output).
//
// Design (MI355X-first, not a translation of the reference's mma.sync tiling):
//  * One wave owns QB blocks of 32 queries. Scores are computed transposed,
//    S^T = K * Q^T, with v_mfma_f32_32x32x16_bf16: A = K rows (from LDS),
//    B = Q^T (resident in VGPRs for the whole kernel). In the 32x32 C layout each
//    lane then holds ONE query (column lane%32) and 16 keys, so the running max
//    and sum are per-lane scalars and the only cross-lane step is one
//    v_permlane32_swap between the two wave halves.
//  * K rows are fed to the score MFMA in a permuted order (bits 2 and 3 of the
//    row index swapped) so that each lane's 16 score registers are exactly the
//    8-key runs the P*V MFMA wants as its B operand: P never leaves registers.
//  * O^T = V^T * P^T with the same MFMA; the V^T operand comes straight from the
//    row-major V tile with ds_read_b64_tr_b16 (gfx950 transposing LDS read), so
//    V needs no transposition pass.
//  * K/V tiles (64 keys) are double-buffered in LDS via global_load_lds_dwordx4
//    (16 B per lane, no VGPR staging), XOR-swizzled in 16-byte chunks against
//    bank conflicts. Work-groups are remapped so one head's query tiles share an
//    XCD (and its L2).
#include "attn_common.hpp"

#ifndef MXA_BF16_NW
#define MXA_BF16_NW 8
#endif
#ifndef MXA_BF16_QB
#define MXA_BF16_QB 1
#endif

namespace mxa {

namespace {

constexpr int D = 128;
constexpr int KT = 64;               // keys per tile
constexpr int ROWB = D * 2;          // bytes per K/V row in LDS
constexpr int TILEB = KT * ROWB;     // bytes per K (or V) tile

// LDS byte offset of 16-byte chunk `lc` of K row `r` (16 chunks per row).
__device__ __forceinline__ int k_off(int r, int lc) { return r * ROWB + ((lc ^ (r & 15)) << 4); }
// LDS byte offset of 16-byte chunk `lc` of V row `r`.
__device__ __forceinline__ int v_off(int r, int lc) { return r * ROWB + ((lc ^ ((r & 3) << 2)) << 4); }

// Score-row -> key permutation inside a 32-key block: swap bits 2 and 3.
__device__ __forceinline__ int perm32(int m) {
  return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1);
}

template <int NW, int QB>
__global__ void __launch_bounds__(NW * 64, 1)
flash_bf16_d128(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                const uint16_t* __restrict__ v, uint16_t* __restrict__ o, mx_attn_params p,
                float c, uint32_t qsign) {
  constexpr int QW = 32 * QB, QT = NW * QW, NT = NW * 64;
  // Two distinct LDS objects (not one array indexed by stage) so the compiler can
  // prove the in-flight global_load_lds into one buffer does not alias reads of the
  // other, and does not wait for the prefetch before every LDS read.
  __shared__ __align__(16) unsigned char lds0[2 * TILEB];
  __shared__ __align__(16) unsigned char lds1[2 * TILEB];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 31, h = lane >> 5;
  const int ntq = (p.Sq + QT - 1) / QT;
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int head = L / ntq, qtile = L % ntq;
  const int kvh = head / (p.Hq / p.Hkv);
  const int q0 = qtile * QT + wave * QW;

  // ---- Q^T fragments (B operand), resident for the whole kernel ----
  bf16x8 qf[QB][8];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    int row = q0 + qb * 32 + n;
    row = row < p.Sq ? row : p.Sq - 1;
    const uint16_t* src = q + int64_t(row) * p.q_stride + head * D + h * 8;
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      u32x4 raw = *reinterpret_cast<const u32x4*>(src + cc * 16);
      raw ^= qsign;  // negative softmax scale: negate Q (exact) and use |scale|
      qf[qb][cc] = __builtin_bit_cast(bf16x8, raw);
    }
  }

  // ---- K/V tile loader: each wave writes 64 consecutive 16-byte LDS slots per op ----
  const int64_t kvbase = int64_t(kvh) * D;
  auto issue = [&](int t, unsigned char* kd) __attribute__((always_inline)) {
    unsigned char* vd = kd + TILEB;
    const int key0 = t * KT;
#pragma unroll
    for (int j = 0; j < (KT * 16) / NT; ++j) {
      const int slot0 = (j * NW + wave) * 64, slot = slot0 + lane;
      const int r = slot >> 4, pc = slot & 15;
      int key = key0 + r;
      key = key < p.Skv ? key : p.Skv - 1;
      const int64_t g = int64_t(key) * p.kv_stride + kvbase;
      g2lds16(k + g + ((pc ^ (r & 15)) << 3), (MXA_LDS void*)(kd + slot0 * 16));
      g2lds16(v + g + ((pc ^ ((r & 3) << 2)) << 3), (MXA_LDS void*)(vd + slot0 * 16));
    }
  };

  f32x16 acc[QB][4];
  float m[QB], l[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m[qb] = -__builtin_inff();
    l[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[qb][db] = f32x16{};
  }

  const int nt = (p.Skv + KT - 1) / KT;
  issue(0, lds0);
  KeyLive live_next = key_live_load(p, lane);

  // Per-lane LDS read offsets that do not depend on the tile.
  int koff[2][8];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const int r = kb * 32 + perm32(n);
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) koff[kb][cc] = k_off(r, 2 * cc + h);
  }
  // ds_read_b64_tr_b16: lane i of a 16-lane group reads 8 bytes of row (i>>2),
  // columns d0 + 4*(i&3); lane j of the group receives column d0+j of those 4 rows.
  const int g16 = lane >> 4, i16 = lane & 15;
  const int trow = (g16 >> 1) * 8 + (i16 >> 2);  // + kc*16 + r*4
  const int tcol = (g16 & 1) * 16 + (i16 & 3) * 4;  // + db*32 (elements)

  auto tile = [&](int t, const unsigned char* kd, unsigned char* nxt) __attribute__((always_inline)) {
    wait_vm();
    __syncthreads();
    const uint64_t live = key_live_ballot(live_next);
    if (t + 1 < nt) {
      issue(t + 1, nxt);
      live_next = key_live_load(p, (t + 1) * KT + lane);
    }
    const unsigned char* vd = kd + TILEB;

    // ---- S^T = K Q^T ----
    f32x16 s[QB][2];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) s[qb][0] = s[qb][1] = f32x16{};
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(kd + koff[kb][cc]);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          s[qb][kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[qb][cc], s[qb][kb], 0, 0, 0);
      }
    }

    // ---- online softmax (base 2), one query per lane ----
    const bool full = live == ~0ull;
    bf16x8 pf[QB][4];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if (!full) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = kb * 32 + (i >> 3) * 16 + h * 8 + (i & 7);
            if (!((live >> key) & 1)) s[qb][kb][i] = -__builtin_inff();
          }
      }
      float mx = s[qb][0][0];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[qb][kb][i]);
      mx = fmaxf(mx, other_half(mx));
      const float mnew = fmaxf(m[qb], mx);
      const float mc = mnew == -__builtin_inff() ? 0.f : mnew * c;
      const float alpha = m[qb] == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(m[qb] * c - mc);
      m[qb] = mnew;
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qb][kb][i], c, -mc));
          s[qb][kb][i] = e;
          rs += e;
        }
      rs += other_half(rs);
      l[qb] = l[qb] * alpha + rs;
      if (!__all(alpha == 1.f)) {
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[qb][db] *= alpha;
      }
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        u32x4 w;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          w[j] = pack_bf16x2(s[qb][kc >> 1][(kc & 1) * 8 + 2 * j], s[qb][kc >> 1][(kc & 1) * 8 + 2 * j + 1]);
        pf[qb][kc] = __builtin_bit_cast(bf16x8, w);
      }
    }

    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const int r0 = kc * 16 + trow, col = db * 32 + tcol;
        const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (MXA_LDS bf16x4*)(vd + v_off(r0, col >> 3) + (col & 7) * 2));
        const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
            (MXA_LDS bf16x4*)(vd + v_off(r0 + 4, col >> 3) + (col & 7) * 2));
        const bf16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          acc[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf[qb][kc], acc[qb][db], 0, 0, 0);
      }
    }
  };
  for (int t = 0; t < nt; t += 2) {
    tile(t, lds0, lds1);
    if (t + 1 < nt) tile(t + 1, lds1, lds0);
  }

  // ---- epilogue: O = acc / l -> bf16 ----
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int row = q0 + qb * 32 + n;
    if (row >= p.Sq) continue;
    const float inv = l[qb] > 0.f ? 1.f / l[qb] : 0.f;
    uint16_t* dst = o + int64_t(row) * p.o_stride + head * D + h * 4;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float* a = reinterpret_cast<const float*>(&acc[qb][db]) + g * 4;
        u32x2 w;
        w[0] = pack_bf16x2(a[0] * inv, a[1] * inv);
        w[1] = pack_bf16x2(a[2] * inv, a[3] * inv);
        uint32_t* d32 = reinterpret_cast<uint32_t*>(dst + db * 32 + g * 8);
        d32[0] = w[0];
        d32[1] = w[1];
      }
  }
}

}  // namespace

// Launch the fast path. Preconditions (checked by the caller): D == 128,
// non-causal, q/k/v 16-byte aligned with token strides % 8 == 0, o 4-byte
// aligned with o_stride % 2 == 0.
hipError_t launch_flash_bf16_d128(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                                  const mx_attn_params& p, hipStream_t s) {
  constexpr int NW = MXA_BF16_NW, QB = MXA_BF16_QB, QT = NW * 32 * QB;
  const float c = __builtin_fabsf(p.scale) * kLog2e;
  const uint32_t qsign = p.scale < 0.f ? 0x80008000u : 0u;
  const int ntq = (p.Sq + QT - 1) / QT;
  const int64_t blocks = int64_t(ntq) * p.Hq;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  const size_t lds = 0;  // static LDS: two 32 KB K/V stages
  hipLaunchKernelGGL((flash_bf16_d128<NW, QB>), dim3(unsigned(blocks)), dim3(NW * 64), lds, s, q, k, v, o, p,
                     c, qsign);
  return hipGetLastError();
}

}  // namespace mxa

// MXFP8 block-scaled GEMM for gfx950: quantizer + GEMM on the MX-scaled MFMA.
// Reference: src/kernels/blockscale.{h,cu} (quantize_blockscaled :113-131,
// quant_kernel MXFP8 branch :69-108, gemm_blockscaled :134-216 on cuBLASLt).
//
// Format (OCP MX, the reference's MXFP8): e4m3 data, one power-of-two scale (UE8M0)
// per 32 consecutive K values of a row. gfx950's v_mfma_scale_f32_32x32x64_f8f6f4
// consumes exactly that: lane half h supplies the UE8M0 scale of K block h of each
// 64-value MFMA step (selected per operand by op_sel); see the operand layout note
// in mxfp8_gemm.
//
// Scale layout: the reference's 128 x 4 interleave (quantizer blockscale.cu:82,
// decoder tests/blockscale_test.cpp:15-17): scale (r, kb) at byte
// (r / 128) kbp 128 + (kb / 4) 512 + (r % 32) 16 + ((r % 128) / 32) 4 + kb % 4,
// kbp = K/32 rounded up to 4, rows padded to 128 (the reference's qscale_bytes size).
// The quantizer writes 127 (= 1.0) into every padding byte, so padded K blocks and
// rows contribute 0 (data 0 times a finite scale) instead of 0 x NaN (0xFF).
//
// GEMM (Y[M,N] bf16 = X[M,K] W[N,K]^T, both K-major): tiles of 256 n x 256 m per
// 4-wave work-group, one wave per SIMD, each wave 128 n x 128 m = 4 x 4 MFMA blocks
// of 32 x 32 (C = W X^T: lane = one m column, 16 n rows; the 256 fp32 accumulators
// live in AGPRs). K advances in stages of 128 bytes DMA'd into LDS
// (buffer_load ... lds, 1 KB per op, rows past the matrix read as zeros), double
// buffered; LDS rows are 128 B with their 16-byte chunks XOR'd by (row >> 1) & 7, so
// each 16-lane group of an operand read hits 16 distinct chunk slots. A stage's
// scales for a lane are one 16-byte load per operand (the interleave puts a 128-row
// band's four 32-row blocks side by side). The bf16 tile leaves through LDS as
// coalesced 16-byte row stores.
#include <type_traits>

#include "attn_common.hpp"

namespace mxa {

namespace {

constexpr int kMxBlock = 32;       // K values per UE8M0 scale
constexpr int kTile = 256;         // n and m per work-group
constexpr int kStage = 128;        // K bytes per LDS stage
constexpr int kStageB = kTile * kStage;  // 32 KB per operand per stage
constexpr int kGroupM = 4;               // tile rows per launch-order group

__host__ __device__ inline int64_t pad_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// ---------------- quantizer ----------------
// One thread per 32-value block of a row: bmax = max |x|; e = the smallest power of
// two with bmax / 2^e <= 448 (frexp of bmax / 448: mantissa 0.5 -> e = ex - 1,
// else ex; clamped to [-127, 127]; bmax = 0 -> -127); q = e4m3(x * 2^-e), round to
// nearest even, saturate to +-448; scale byte e + 127 (reference :95-104).
__global__ void __launch_bounds__(256) mxfp8_quant(const uint16_t* __restrict__ x, int64_t ldx, int64_t rows,
                                                   int64_t K, uint8_t* __restrict__ q, uint8_t* __restrict__ sf,
                                                   int64_t kbp, int64_t rows_pad) {
  const int64_t nkb = K / kMxBlock;
  const int64_t id = int64_t(blockIdx.x) * 256 + threadIdx.x;  // over rows_pad * kbp
  if (id >= rows_pad * kbp) return;
  const int64_t r = id / kbp, kb = id % kbp;
  // the reference's 128 x 4 interleaved scale layout (blockscale.cu:82)
  const int64_t so = (r / 128) * kbp * 128 + (kb / 4) * 512 + (r % 32) * 16 + (r % 128) / 32 * 4 + kb % 4;
  if (r >= rows || kb >= nkb) {  // padding: scale 1.0
    sf[so] = 127;
    return;
  }
  const uint16_t* src = x + r * ldx + kb * kMxBlock;
  float v[32];
  float bmax = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const u32x4 u = *reinterpret_cast<const u32x4*>(src + 8 * j);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      v[8 * j + t] = bf2f(uint16_t(u[t >> 1] >> ((t & 1) * 16)));
      bmax = fmaxf(bmax, fabsf(v[8 * j + t]));
    }
  }
  int e = -127;
  if (bmax > 0.f) {
    int ex;
    const float mant = frexpf(bmax / 448.f, &ex);
    e = mant == 0.5f ? ex - 1 : ex;
    e = e < -127 ? -127 : (e > 127 ? 127 : e);
  }
  const float inv = exp2f(float(-e));
  u32x4 w[2];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float a = __builtin_fminf(__builtin_fmaxf(v[4 * j] * inv, -448.f), 448.f);
    float b = __builtin_fminf(__builtin_fmaxf(v[4 * j + 1] * inv, -448.f), 448.f);
    float c = __builtin_fminf(__builtin_fmaxf(v[4 * j + 2] * inv, -448.f), 448.f);
    float d = __builtin_fminf(__builtin_fmaxf(v[4 * j + 3] * inv, -448.f), 448.f);
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w[j >> 2][j & 3] = uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true));
  }
  u32x4* dst = reinterpret_cast<u32x4*>(q + r * K + kb * kMxBlock);
  dst[0] = w[0];
  dst[1] = w[1];
  sf[so] = uint8_t(e + 127);
}

// ---------------- GEMM ----------------
// One operand's DMA of stage k0: 32 ops of 1 KB (8 rows x 128 B each); wave w
// issues ops j = 4 * jj + w. Lane i of op j fills physical chunk i % 8 of row
// 8 j + i / 8, i.e. logical chunk (i % 8) ^ ((row >> 1) & 7); ((row >> 1) & 7)
// depends on j only through its parity, which is the wave's. Both operands have
// row stride K, so one set of 8 per-lane offsets serves both and the only
// scalar offset is k0.
struct OpAddr {
  uint32_t vo[8];  // row (8 j + lane / 8) * K + logical chunk * 16, j = 4 jj + wave
  uint32_t chunk;  // logical chunk * 16 (for the K-tail check)
};
__device__ __forceinline__ OpAddr op_addr(int64_t K, int lane, int wave) {
  OpAddr a;
  const int rin = lane >> 3, p = lane & 7;
  const int row = 8 * (wave & 1) + rin;  // row modulo 16 is what the swizzle sees
  const int c = p ^ ((row >> 1) & 7);
  a.chunk = uint32_t(c * 16);
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) a.vo[jj] = uint32_t(8 * (4 * jj + wave) + rin) * uint32_t(K) + a.chunk;
  return a;
}

// Lanes whose chunk lies past K read zeros (an offset past the buffer's range);
// for a stage wholly past K every lane does, and the DMA only clears LDS.
__device__ __forceinline__ void dma_stage(__amdgpu_buffer_rsrc_t rs, const OpAddr& a, int64_t K, int k0,
                                          unsigned char* dst, int wave) {
  const bool past = uint32_t(k0) + a.chunk >= uint32_t(K);
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) {
    const int j = 4 * jj + wave;
    const uint32_t off = past ? 0x80000000u : a.vo[jj];
    buf2lds16(rs, off, uint32_t(k0), (MXA_LDS void*)(dst + j * 1024));
  }
}

// Epilogue through LDS: the 256 x 256 bf16 Y tile (row m = 512 B of n) fills the
// stage buffers. Lane (m = lane % 32 of block j, h = lane / 32) holds n = 8g + 4h +
// (0..3) of block i; 16-byte chunk q of row m sits at q ^ (m % 16), so the 8-byte
// writes and the 16-byte row reads are free of bank conflicts, and each row goes out
// as coalesced 16-byte stores. ALPHA: Y = alpha * C (+ Y).
template <bool ALPHA>
__device__ __forceinline__ void store_tile(const f32x16 (&acc)[4][4], unsigned char* lds, uint16_t* __restrict__ y,
                                           int64_t ldy, int M, int N, int m0, int n0, int wm, int wn, int lane,
                                           int beta, float alpha) {
  const int n = lane & 31, h = lane >> 5;
  block_sync();  // every wave is done with the operand buffers
  {
    const int xs = lane & 15;  // m % 16 (wm and 32 j are multiples of 16)
    unsigned char* wp = lds + (wm + n) * 512 + 8 * h + wn * 2;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int cs = ((4 * i + g) ^ xs) << 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x16& c = acc[i][j];
          float v[4] = {c[4 * g], c[4 * g + 1], c[4 * g + 2], c[4 * g + 3]};
          if constexpr (ALPHA) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] *= alpha;
          }
          if (beta) {  // Y += C with one rounding: add the old values in fp32 here
            const int m = m0 + wm + 32 * j + n, nb = n0 + wn + 32 * i + 8 * g + 4 * h;
            if (m < M) {
              const uint16_t* p = y + int64_t(m) * ldy + nb;
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (nb + e < N) v[e] += bf2f(p[e]);
            }
          }
          *reinterpret_cast<u32x2*>(wp + j * 32 * 512 + cs) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        }
      }
  }
  block_sync();
  const bool vec = (reinterpret_cast<uintptr_t>(y) & 15) == 0 && ldy % 8 == 0;
  const int c = threadIdx.x & 31, nn = n0 + 8 * c;
#pragma unroll 4
  for (int it = 0; it < 32; ++it) {
    const int r = it * 8 + (threadIdx.x >> 5), m = m0 + r;
    if (m >= M) break;
    const u32x4 v = *reinterpret_cast<const u32x4*>(lds + r * 512 + ((c ^ (r & 15)) << 4));
    uint16_t* p = y + int64_t(m) * ldy + nn;
    if (vec && nn + 7 < N) {
      *reinterpret_cast<u32x4*>(p) = v;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (nn + e < N) p[e] = uint16_t(v[e >> 1] >> ((e & 1) * 16));
    }
  }
}

__global__ void __launch_bounds__(256, 1)
mxfp8_gemm(const uint8_t* __restrict__ wq, const uint8_t* __restrict__ wsf, const uint8_t* __restrict__ xq,
           const uint8_t* __restrict__ xsf, uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K, int beta,
           int ntn, int ntm) {
  __shared__ __align__(16) unsigned char lds[4 * kStageB];
  // stage buffers: operand A at lds + (st % 2) * kStageB, operand B 64 KB above it
  unsigned char *const a0 = lds, *const a1 = lds + kStageB, *const b0 = lds + 2 * kStageB;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  // grouped order: consecutive tiles walk kGroupM tile rows (m) before moving
  // along n, so the 32 concurrent tiles of one XCD (one L2) form a 4 x 8 block
  // and share 12 operand strips instead of 33
  const int gsz = kGroupM * ntn, grp = L / gsz, fm = grp * kGroupM;
  const int gm = min(ntm - fm, kGroupM), li = L - grp * gsz;
  const int tm = fm + li % gm, tn = li / gm;
  const int n0 = tn * kTile, m0 = tm * kTile;
  const int wn = (wave & 1) * 128, wm = (wave >> 1) * 128;
  const int kbp = int(pad_up(K / kMxBlock, 4));
  const int nst = (K + kStage - 1) / kStage;

  const __amdgpu_buffer_rsrc_t rw = buf_rsrc(wq + int64_t(n0) * K, uint32_t(int64_t(N - n0) * K));
  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(xq + int64_t(m0) * K, uint32_t(int64_t(M - m0) * K));
  const OpAddr oa = op_addr(K, lane, wave_u);
  // Scales, in the reference's 128 x 4 interleaved layout: byte (r / 128) kbp 128 +
  // (kb / 4) 512 + (r % 32) 16 + ((r % 128) / 32) 4 + kb % 4. A wave's 128 rows are one
  // 128-row band, so lane n's four row blocks (r % 32 = n, (r % 128) / 32 = b) for the
  // four K blocks of stage st (kb / 4 = st) are the 16 contiguous bytes at
  // band + st 512 + 16 n: one 16-byte load per operand per stage. Bands past the
  // 128-padded matrix read as zeros (their data is zero too).
  const int n = lane & 31, h = lane >> 5;
  const __amdgpu_buffer_rsrc_t rsw = buf_rsrc(wsf, uint32_t(pad_up(N, 128) * kbp));
  const __amdgpu_buffer_rsrc_t rsx = buf_rsrc(xsf, uint32_t(pad_up(M, 128) * kbp));
  const uint32_t sw_off = uint32_t((n0 + wn) / 128) * uint32_t(kbp) * 128u + uint32_t(16 * n);
  const uint32_t sx_off = uint32_t((m0 + wm) / 128) * uint32_t(kbp) * 128u + uint32_t(16 * n);
  // raw scale words of stage st (word b = row block b), loaded a stage ahead and
  // unpacked only after the next stage's wait, so no stage waits on their latency
  auto scales = [&](int st, uint32_t (&ra)[4], uint32_t (&rb)[4]) __attribute__((always_inline)) {
    const u32x4 wa = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsw, sw_off + uint32_t(st * 512), 0, 0));
    const u32x4 wb = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsx, sx_off + uint32_t(st * 512), 0, 0));
#pragma unroll
    for (int b = 0; b < 4; ++b) ra[b] = wa[b], rb[b] = wb[b];
  };

  // LDS operand reads: rows row0 + n of an operand tile for K step s. In the f8
  // operand of the 32x32x64 MFMA, bytes 0-15 of lane half h are K 16h .. 16h+15 and
  // bytes 16-31 are K 32 + 16h ..; the UE8M0 scale of lane half h applies to K block
  // h (K 32h .. 32h+31, i.e. bytes 0-15 of both halves for h = 0, bytes 16-31 for
  // h = 1). So lane half h takes logical chunks 4s + h (K block 2s) and 4s + 2 + h
  // (K block 2s + 1), and its scale is that of K block 2s + h. The per-lane part of
  // the address is one base plus the chunk offsets; the row block is a constant.
  const int x = (n >> 1) & 7;
  int coff[4];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    coff[2 * s] = ((4 * s + h) ^ x) << 4;
    coff[2 * s + 1] = ((4 * s + 2 + h) ^ x) << 4;
  }
  const int abase = (wn + n) * kStage, bbase = (wm + n) * kStage;
  auto opread = [&](const unsigned char* base, int b, int s) __attribute__((always_inline)) -> i32x8 {
    const unsigned char* rp = base + b * 32 * kStage;
    const i32x4 lo = *reinterpret_cast<const i32x4*>(rp + coff[2 * s]);
    const i32x4 hi = *reinterpret_cast<const i32x4*>(rp + coff[2 * s + 1]);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // opaque zeros: left as constants, the register allocator splits the
      // accumulators' live ranges at the loop header and spills them
      acc[i][j] = f32x16{};
      asm volatile("" : "+a"(acc[i][j]));
    }

  // DMA of stage st (operands and the raw scale words) into buffers (da, db)
  auto fetch = [&](int st, unsigned char* da, unsigned char* db, uint32_t (&ra)[4],
                   uint32_t (&rb)[4]) __attribute__((always_inline)) {
    dma_stage(rw, oa, K, st * kStage, da, wave_u);
    dma_stage(rx, oa, K, st * kStage, db, wave_u);
    scales(st, ra, rb);
  };
  // byte 0: K block 2s + h of step s = 0, byte 2: of step s = 1 (op_sel 0 / 2)
  auto unpack = [&](const uint32_t (&ra)[4], const uint32_t (&rb)[4], uint32_t (&ta)[4],
                    uint32_t (&tb)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < 4; ++b) ta[b] = (ra[b] >> (8 * h)) & 0x00FF00FFu, tb[b] = (rb[b] >> (8 * h)) & 0x00FF00FFu;
  };
  auto rd = [&](const unsigned char* ca, const unsigned char* cb, auto sc, i32x8 (&av)[4],
                i32x8 (&bv)[4]) __attribute__((always_inline)) {
    constexpr int S = decltype(sc)::value;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      av[b] = opread(ca + abase, b, S);
      bv[b] = opread(cb + bbase, b, S);
    }
  };
  // operands stay in VGPRs (the 256 accumulators fill the AGPR file); the pin
  // is also where the reads are waited for
  auto pin = [&](i32x8 (&av)[4], i32x8 (&bv)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < 4; ++b) asm volatile("" : "+v"(av[b]), "+v"(bv[b]));
  };
  // MFMAs [lo, hi) of a K step, in (i, j) order
  auto mm = [&](const i32x8 (&av)[4], const i32x8 (&bv)[4], const uint32_t (&ta)[4], const uint32_t (&tb)[4],
                auto sc, auto lo, auto hi) __attribute__((always_inline)) {
    constexpr int S = decltype(sc)::value;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (4 * i + j >= decltype(lo)::value && 4 * i + j < decltype(hi)::value)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av[i], bv[j], acc[i][j], 0, 0, 2 * S,
                                                                     int(ta[i]), 2 * S, int(tb[j]));
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;

  // Software pipeline: the LDS reads of the next K step are in flight while the
  // current step's 16 MFMAs run. Stage st + 2 is DMA'd into stage st's buffers
  // once every wave has read them (the barrier after the step-1 reads).
  uint32_t ra[4], rb[4], ta[4], tb[4];
  i32x8 r0a[4], r0b[4], r1a[4], r1b[4];
  fetch(0, a0, b0, ra, rb);
  wait_vm();
  block_sync();
  unpack(ra, rb, ta, tb);
  fetch(1, a1, b0 + kStageB, ra, rb);
  rd(a0, b0, S0{}, r0a, r0b);
  pin(r0a, r0b);

  using C0 = std::integral_constant<int, 0>;
  using C2 = std::integral_constant<int, 2>;
  using C16 = std::integral_constant<int, 16>;
  // Stage body. Step 0's MFMAs are interleaved with step 1's LDS reads; two of
  // step 1's MFMAs are issued before the stage barrier so the matrix unit stays
  // busy while the wave waits there; the remaining 14 are interleaved with the
  // DMA of stage st + 2 (unconditional: a stage past K only clears LDS that is
  // never read) and with the LDS reads of the next stage's step 0 (on the last
  // stage they fetch stale data that is never used).
  auto stage = [&](int st, unsigned char* ca, unsigned char* cb, const unsigned char* na,
                   const unsigned char* nb) __attribute__((always_inline)) {
    rd(ca, cb, S1{}, r1a, r1b);
    mm(r0a, r0b, ta, tb, S0{}, C0{}, C16{});
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    }
    __builtin_amdgcn_sched_barrier(0);
    pin(r1a, r1b);
    mm(r1a, r1b, ta, tb, S1{}, C0{}, C2{});
    __builtin_amdgcn_sched_barrier(0);
    uint32_t tn[4], tm[4];
    wait_vm();     // this wave's DMA of stage st+1 (and its scale words) landed ...
    block_sync();  // ... for every wave, and every wave has read stage st
    unpack(ra, rb, tn, tm);
    fetch(st + 2, ca, cb, ra, rb);
    rd(na, nb, S0{}, r0a, r0b);
    mm(r1a, r1b, ta, tb, S1{}, C2{}, C16{});
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // VMEM: DMA, scale loads
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
    }
    __builtin_amdgcn_sched_barrier(0);
    pin(r0a, r0b);
#pragma unroll
    for (int b = 0; b < 4; ++b) ta[b] = tn[b], tb[b] = tm[b];
  };
  for (int st = 0; st < nst; st += 2) {
    stage(st, a0, b0, a1, b0 + kStageB);
    if (st + 1 < nst) stage(st + 1, a1, b0 + kStageB, a0, b0);
  }
  wait_vm();  // no LDS-DMA may land after the work-group ends

  store_tile<false>(acc, lds, y, ldy, M, N, m0, n0, wm, wn, lane, beta, 1.f);
}


// ---------------- NVFP4 ----------------
// Format (the reference's NVFP4, blockscale.cu:36-93): e2m1 data, two per byte (the
// lower-index value in the low nibble), one e4m3 scale per 16 consecutive K values of
// a row (the same 128 x 4 interleave with K/16 blocks, padding bytes 0, as the
// reference's memset), and a per-tensor amax: g = amax / (6 * 448), block scale
// se = e4m3(bmax / (6 g)), codes e2m1(x / (se g)). The GEMM returns
// alpha * sum (e2m1 se)_X (e2m1 se)_W with alpha = gW gX.
constexpr int kFp4Block = 16;
constexpr float kFp4Range = 6.f * 448.f;

__global__ void nvfp4_amax_init(float* amax) {
  if (threadIdx.x == 0) *amax = 0.f;
}

// max |x| of the tensor (reference amax_kernel :45-67): a 1024-thread work-group per
// range of rows, four 16-byte loads in flight per thread, a wave max, the work-group
// max through LDS, one atomic max per work-group on the value's bits (non-negative
// floats order as integers). At most 256 work-groups: atomics on one address
// serialise (one per wave cost ~40 us at 4096 x 4096).
__global__ void __launch_bounds__(1024) nvfp4_amax(const uint16_t* __restrict__ x, int64_t ldx, int64_t rows,
                                                   int64_t K, float* amax) {
  const int64_t nv = K / 8;
  const int64_t per = (rows + gridDim.x - 1) / gridDim.x;
  const int64_t r0 = int64_t(blockIdx.x) * per, r1 = r0 + per < rows ? r0 + per : rows;
  const int64_t n = r1 > r0 ? (r1 - r0) * nv : 0;
  float m = 0.f;
  for (int64_t i0 = threadIdx.x; i0 < n; i0 += 4 * 1024) {
    u32x4 u[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int64_t i = i0 + k * 1024;
      const int64_t r = r0 + i / nv, j = i - (i / nv) * nv;
      u[k] = i < n ? *reinterpret_cast<const u32x4*>(x + r * ldx + 8 * j) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int t = 0; t < 8; ++t) m = fmaxf(m, fabsf(bf2f(uint16_t(u[k][t >> 1] >> ((t & 1) * 16)))));
  }
#pragma unroll
  for (int o = 32; o; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  __shared__ float wmax[16];
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < 16; ++w) m = fmaxf(m, wmax[w]);
    atomicMax(reinterpret_cast<int*>(amax), __float_as_int(m));
  }
}

// One thread per 16-value block of a row (reference quant_kernel NVFP4 branch :76-93);
// padding scale bytes get 0.
__global__ void __launch_bounds__(256) nvfp4_quant(const uint16_t* __restrict__ x, int64_t ldx, int64_t rows,
                                                   int64_t K, uint8_t* __restrict__ q, uint8_t* __restrict__ sf,
                                                   const float* __restrict__ amax, int64_t kbp, int64_t rows_pad) {
  const int64_t nkb = K / kFp4Block;
  const int64_t id = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (id >= rows_pad * kbp) return;
  const int64_t r = id / kbp, kb = id % kbp;
  const int64_t so = (r / 128) * kbp * 128 + (kb / 4) * 512 + (r % 32) * 16 + (r % 128) / 32 * 4 + kb % 4;
  if (r >= rows || kb >= nkb) {
    sf[so] = 0;
    return;
  }
  const uint16_t* src = x + r * ldx + kb * kFp4Block;
  float v[16];
  float bmax = 0.f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const u32x4 u = *reinterpret_cast<const u32x4*>(src + 8 * j);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      v[8 * j + t] = bf2f(uint16_t(u[t >> 1] >> ((t & 1) * 16)));
      bmax = fmaxf(bmax, fabsf(v[8 * j + t]));
    }
  }
  const float a = *amax;
  const float g = a > 0.f ? a / kFp4Range : 1.f;
  const float inv6g = 1.f / (6.f * g);
  // e4m3 of bmax / (6 g), saturating: clamp to 448, then round to nearest even
  const float t = __builtin_fminf(bmax * inv6g, 448.f);
  const uint32_t se = uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(t, t, 0, false)) & 0xffu;
  const float sd = __builtin_amdgcn_cvt_f32_fp8(int(se), 0) * g;
  const float inv = sd > 0.f ? 1.f / sd : 0.f;
  // e2m1 codes: v_cvt_scalef32_pk_fp4_f32 (scale 1) rounds to the nearest magnitude of
  // {0, 0.5, 1, 1.5, 2, 3, 4, 6} with ties to the even code, saturates at 6 and sets the
  // sign bit for negative values: the reference's threshold sum (:38-42), checked on
  // the device against it over 2M value pairs (every midpoint +-1 ulp, -0, saturation);
  // two values per byte, the lower-index one in the low nibble
  u32x2 w = {0u, 0u};
  static_for<8>([&](auto jc) __attribute__((always_inline)) {
    constexpr int j = decltype(jc)::value;
    w[j >> 2] = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w[j >> 2], v[2 * j] * inv, v[2 * j + 1] * inv, 1.f, j & 3);
  });
  *reinterpret_cast<u32x2*>(q + (r * K + kb * kFp4Block) / 2) = w;
  sf[so] = uint8_t(se);
}

// NVFP4 GEMM: the MXFP8 kernel's tiling (256 n x 256 m per 4-wave work-group, 128 x 128
// per wave, 256 fp32 accumulators in AGPRs, K stages of 128 bytes = 256 values DMA'd
// into LDS with the same swizzle, XCD-grouped tile order, LDS epilogue), but the raw e2m1
// data is dequantized in registers and multiplied on the f16 MFMA (32x32x16). gfx950's
// scaled MFMA takes one power-of-two scale per 32 values, NVFP4 an e4m3 scale per 16;
// the product of an e2m1 value and an e4m3 scale has at most 5 significant bits, so
// e2m1 -> f16 (v_cvt_scalef32_pk_f16_fp4, scale 1) times the block scale in f16
// (v_pk_mul_f16) is exact, as are the MFMA's f16 products; accumulation is fp32, and
// alpha = gW gX scales the tile in the epilogue.
//
// Operand layout: the MFMA sums its 16 K values in any order, so the two lane halves
// take different 16-value blocks: for 32-value chunk c of a stage, lane half h of row
// r reads the 8 bytes of block 2c + h (one ds_read_b64) and feeds values 0-7 of it to
// MFMA step 2c and values 8-15 to step 2c + 1; W and X use the same assignment, so
// every product pairs the same K. One e4m3 scale per lane per chunk and operand block.
using f16x2 = __attribute__((ext_vector_type(2))) _Float16;
using f16x8 = __attribute__((ext_vector_type(8))) _Float16;

__device__ __forceinline__ f16x8 fp4x8_to_f16(uint32_t d, f16x2 s) {
  const f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, 1.f, 0) * s;
  const f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, 1.f, 1) * s;
  const f16x2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, 1.f, 2) * s;
  const f16x2 e = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, 1.f, 3) * s;
  return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], e[0], e[1]};
}

__global__ void __launch_bounds__(256, 1)
nvfp4_gemm(const uint8_t* __restrict__ wq, const uint8_t* __restrict__ wsf, const float* __restrict__ wamax,
           const uint8_t* __restrict__ xq, const uint8_t* __restrict__ xsf, const float* __restrict__ xamax,
           uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K, int beta, int ntn, int ntm) {
  __shared__ __align__(16) unsigned char lds[4 * kStageB];
  // stage buffers: operand W at lds + bi * kStageB, operand X at lds + (2 + bi) * kStageB
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int L = xcd_remap(blockIdx.x, gridDim.x);
  const int gsz = kGroupM * ntn, grp = L / gsz, fm = grp * kGroupM;
  const int gm = min(ntm - fm, kGroupM), li = L - grp * gsz;
  const int tm = fm + li % gm, tn = li / gm;
  const int n0 = tn * kTile, m0 = tm * kTile;
  const int wn = (wave & 1) * 128, wm = (wave >> 1) * 128;
  const int RB = K / 2;                                  // bytes per row
  const int kbp = int(pad_up(K / kFp4Block, 4));
  const int nst = (RB + kStage - 1) / kStage;            // stages of 256 values

  const __amdgpu_buffer_rsrc_t rw = buf_rsrc(wq + int64_t(n0) * RB, uint32_t(int64_t(N - n0) * RB));
  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(xq + int64_t(m0) * RB, uint32_t(int64_t(M - m0) * RB));
  const OpAddr oa = op_addr(RB, lane, wave_u);
  // Scales: a wave's 128 rows are one 128-row band; lane n's bytes for row blocks b =
  // 0..3 (r % 32 = n, (r % 128) / 32 = b) and K blocks 4t..4t+3 are the 16 bytes at
  // band + t 512 + 16 n (word b, byte kb % 4). A stage's 16 blocks: 4 loads per operand.
  const int n = lane & 31, h = lane >> 5;
  const __amdgpu_buffer_rsrc_t rsw = buf_rsrc(wsf, uint32_t(pad_up(N, 128) * kbp));
  const __amdgpu_buffer_rsrc_t rsx = buf_rsrc(xsf, uint32_t(pad_up(M, 128) * kbp));
  const uint32_t sw_off = uint32_t((n0 + wn) / 128) * uint32_t(kbp) * 128u + uint32_t(16 * n);
  const uint32_t sx_off = uint32_t((m0 + wm) / 128) * uint32_t(kbp) * 128u + uint32_t(16 * n);
  auto fetch = [&](int st, int bi, u32x4 (&sa)[4], u32x4 (&sb)[4]) __attribute__((always_inline)) {
    dma_stage(rw, oa, RB, st * kStage, lds + bi * kStageB, wave_u);
    dma_stage(rx, oa, RB, st * kStage, lds + (2 + bi) * kStageB, wave_u);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      sa[t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsw, sw_off + uint32_t((4 * st + t) * 512), 0, 0));
      sb[t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsx, sx_off + uint32_t((4 * st + t) * 512), 0, 0));
    }
  };
  // LDS read address of (row block b, chunk c): row (w* + 32 b + n), logical 16-byte
  // chunk c at physical c ^ ((row >> 1) & 7), this half's 8 bytes
  const int x = (n >> 1) & 7;
  const int abase = (wn + n) * kStage + 8 * h, bbase = (wm + n) * kStage + 8 * h;
  // the block scale of (row block b, chunk c) in f16, both halves of the pair
  auto scale_of = [&](const u32x4 (&sw)[4], int b, int c) __attribute__((always_inline)) -> f16x2 {
    const uint32_t byte = (sw[c >> 1][b] >> (8 * (2 * (c & 1) + h))) & 0xffu;
    const float f = __builtin_amdgcn_cvt_f32_fp8(int(byte), 0);
    return __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(f, f));
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[i][j] = f32x16{};
      asm volatile("" : "+a"(acc[i][j]));
    }

  u32x4 sa[4], sb[4], na[4], nb[4];
  fetch(0, 0, na, nb);
  for (int st = 0; st < nst; ++st) {
    const int bi = st & 1;
    wait_vm();     // this wave's DMA of stage st and its scale words landed ...
    block_sync();  // ... for every wave, and every wave is done with stage st - 1
#pragma unroll
    for (int t = 0; t < 4; ++t) sa[t] = na[t], sb[t] = nb[t];
    if (st + 1 < nst) fetch(st + 1, bi ^ 1, na, nb);
    const unsigned char* ca = lds + bi * kStageB;
    const unsigned char* cb = lds + (2 + bi) * kStageB;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      u32x2 ra[4], rb[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int co = ((c ^ x) << 4) + b * 32 * kStage;
        ra[b] = *reinterpret_cast<const u32x2*>(ca + abase + co);
        rb[b] = *reinterpret_cast<const u32x2*>(cb + bbase + co);
      }
      f16x2 psa[4], psb[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) psa[b] = scale_of(sa, b, c), psb[b] = scale_of(sb, b, c);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        f16x8 av[4], bv[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) av[b] = fp4x8_to_f16(ra[b][u], psa[b]), bv[b] = fp4x8_to_f16(rb[b][u], psb[b]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
      }
    }
  }
  wait_vm();  // no LDS-DMA may land after the work-group ends
  const float aw = *wamax, ax = *xamax;
  const float alpha = (aw > 0.f ? aw / kFp4Range : 1.f) * (ax > 0.f ? ax / kFp4Range : 1.f);
  store_tile<true>(acc, lds, y, ldy, M, N, m0, n0, wm, wn, lane, beta, alpha);
}

}  // namespace

size_t mx_qscale_size(int64_t rows, int64_t K) { return size_t(pad_up(rows, 128) * pad_up(K / kMxBlock, 4)); }

hipError_t launch_mxfp8_quant(const uint16_t* x, int64_t ldx, int64_t rows, int64_t K, uint8_t* q, uint8_t* sf,
                              hipStream_t s) {
  const int64_t kbp = pad_up(K / kMxBlock, 4), rp = pad_up(rows, 128);
  const int64_t blocks = (rp * kbp + 255) / 256;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(mxfp8_quant, dim3(unsigned(blocks)), dim3(256), 0, s, x, ldx, rows, K, q, sf, kbp, rp);
  return hipGetLastError();
}

// Preconditions (checked by the caller): K % 32 == 0, (N + 255) / 256 * 256 * K < 2^31,
// same for M; beta 0 or 1.
hipError_t launch_mxfp8_gemm(const uint8_t* wq, const uint8_t* wsf, const uint8_t* xq, const uint8_t* xsf,
                             uint16_t* y, int64_t ldy, int M, int N, int K, int beta, hipStream_t s) {
  const int ntn = (N + kTile - 1) / kTile, ntm = (M + kTile - 1) / kTile;
  const int64_t blocks = int64_t(ntn) * ntm;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(mxfp8_gemm, dim3(unsigned(blocks)), dim3(256), 0, s, wq, wsf, xq, xsf, y, ldy, M, N, K, beta,
                     ntn, ntm);
  return hipGetLastError();
}

hipError_t launch_nvfp4_quant(const uint16_t* x, int64_t ldx, int64_t rows, int64_t K, uint8_t* q, uint8_t* sf,
                              float* amax, hipStream_t s) {
  const int64_t kbp = pad_up(K / kFp4Block, 4), rp = pad_up(rows, 128);
  const int64_t blocks = (rp * kbp + 255) / 256;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(nvfp4_amax_init, dim3(1), dim3(64), 0, s, amax);
  hipLaunchKernelGGL(nvfp4_amax, dim3(unsigned(rows < 256 ? rows : 256)), dim3(1024), 0, s, x, ldx, rows, K, amax);
  hipLaunchKernelGGL(nvfp4_quant, dim3(unsigned(blocks)), dim3(256), 0, s, x, ldx, rows, K, q, sf,
                     (const float*)amax, kbp, rp);
  return hipGetLastError();
}

// Preconditions (checked by the caller): K % 32 == 0, (N + 255) / 256 * 256 * K / 2 < 2^31,
// same for M; beta 0 or 1; the amax pointers are device floats written by the quantizer.
hipError_t launch_nvfp4_gemm(const uint8_t* wq, const uint8_t* wsf, const float* wamax, const uint8_t* xq,
                             const uint8_t* xsf, const float* xamax, uint16_t* y, int64_t ldy, int M, int N, int K,
                             int beta, hipStream_t s) {
  const int ntn = (N + kTile - 1) / kTile, ntm = (M + kTile - 1) / kTile;
  const int64_t blocks = int64_t(ntn) * ntm;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(nvfp4_gemm, dim3(unsigned(blocks)), dim3(256), 0, s, wq, wsf, wamax, xq, xsf, xamax, y, ldy, M,
                     N, K, beta, ntn, ntm);
  return hipGetLastError();
}

}  // namespace mxa

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

  // epilogue through LDS: the 256 x 256 bf16 Y tile (row m = 512 B of n) fills
  // the stage buffers. Lane (m = lane % 32 of block j, h = lane / 32) holds n =
  // 8g + 4h + (0..3) of block i; 16-byte chunk q of row m sits at q ^ (m % 16), so
  // the 8-byte writes and the 16-byte row reads are free of bank conflicts, and
  // each row goes out as coalesced 16-byte stores.
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

}  // namespace mxa

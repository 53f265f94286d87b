// head_norm_rope for gfx950: per-head RMS-norm + rotary embedding, written to
// dense [S, H, D] bf16. Reference: src/kernels/ops.cu:87-119 (kernel), :197-210
// (launcher), src/kernels/ops.h:30-41 (contract). HBM-bound: one wave per
// (token, head) row, four rows per work-group.
#include "norm_rope.hpp"

namespace mxa {

namespace {

template <int NJ>
__global__ void __launch_bounds__(256) head_norm_rope_kernel(const uint16_t* __restrict__ in, int64_t S,
                                                             int64_t in_stride, int64_t col0, int H, int D,
                                                             NormRope nr, uint16_t* __restrict__ out) {
  __shared__ float buf[4][64 * NJ];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t rowid = int64_t(blockIdx.x) * 4 + wave;  // = s * H + h
  if (rowid >= S * H) return;
  const int64_t s = rowid / H;
  const int h = int(rowid % H);
  const uint16_t* src = in + s * in_stride + col0 + int64_t(h) * D;
  float v[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int d = nr_channel<NJ>(j, lane);
    v[j] = d < D ? bf2f(src[d]) : 0.f;
  }
  uint16_t r[NJ];
  norm_rope_row<NJ>(v, r, D, s, nr, buf[wave], lane);
  uint16_t* dst = out + rowid * D;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int d = nr_channel<NJ>(j, lane);
    if (d < D) dst[d] = r[j];
  }
}

// D = 128: one row per 16 lanes (nr128_row), 16 rows per work-group, 16-byte
// loads and stores. Requires 16-byte aligned rows (in, in_stride, col0, out).
template <int MODE>
__global__ void __launch_bounds__(256) head_norm_rope_d128(const uint16_t* __restrict__ in, int64_t S,
                                                           int64_t in_stride, int64_t col0, int H, NormRope nr,
                                                           uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t rowid = int64_t(blockIdx.x) * 16 + (threadIdx.x >> 4);  // = s * H + h
  const bool valid = rowid < S * H;
  const int64_t s = valid ? rowid / H : 0;
  const int h = valid ? int(rowid % H) : 0;
  float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (valid) load8_bf16(x, in + s * in_stride + col0 + int64_t(h) * 128 + 8 * (lane & 15));
  nr128_row<MODE>(x, s, valid, nr, lane);
  if (valid) *reinterpret_cast<u32x4*>(out + rowid * 128 + 8 * (lane & 15)) = pack8_bf16(x);
}

}  // namespace

hipError_t launch_head_norm_rope(const uint16_t* in, int64_t S, int64_t in_stride, int64_t col0, int H, int D,
                                 const NormRope& nr, uint16_t* out, hipStream_t s) {
  const int64_t rows = S * H;
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid{unsigned(blocks)}, block{256};
  const bool a16 = (reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) % 16 == 0 &&
                   in_stride % 8 == 0 && col0 % 8 == 0;
  if (D == 128 && a16 && nr128_supported(nr, S)) {
    const int64_t b16 = (rows + 15) / 16;
    if (b16 > 0x7fffffff) return hipErrorInvalidValue;
    const int m = nr128_mode(nr);
    auto kern = m == kRopeNone ? head_norm_rope_d128<kRopeNone>
              : m == kRopeInterleaved ? head_norm_rope_d128<kRopeInterleaved> : head_norm_rope_d128<kRopeHalf>;
    hipLaunchKernelGGL(kern, dim3(unsigned(b16)), block, 0, s, in, S, in_stride, col0, H, nr, out);
    return hipGetLastError();
  }
  if (D <= 64) hipLaunchKernelGGL(head_norm_rope_kernel<1>, grid, block, 0, s, in, S, in_stride, col0, H, D, nr, out);
  else if (D <= 128) hipLaunchKernelGGL(head_norm_rope_kernel<2>, grid, block, 0, s, in, S, in_stride, col0, H, D, nr, out);
  else if (D <= 192) hipLaunchKernelGGL(head_norm_rope_kernel<3>, grid, block, 0, s, in, S, in_stride, col0, H, D, nr, out);
  else hipLaunchKernelGGL(head_norm_rope_kernel<4>, grid, block, 0, s, in, S, in_stride, col0, H, D, nr, out);
  return hipGetLastError();
}

}  // namespace mxa

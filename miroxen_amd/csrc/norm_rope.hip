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

}  // namespace

hipError_t launch_head_norm_rope(const uint16_t* in, int64_t S, int64_t in_stride, int64_t col0, int H, int D,
                                 const NormRope& nr, uint16_t* out, hipStream_t s) {
  const int64_t rows = S * H;
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid{unsigned(blocks)}, block{256};
  if (D <= 64) hipLaunchKernelGGL(head_norm_rope_kernel<1>, grid, block, 0, s, in, S, in_stride, col0, H, D, nr, out);
  else if (D <= 128) hipLaunchKernelGGL(head_norm_rope_kernel<2>, grid, block, 0, s, in, S, in_stride, col0, H, D, nr, out);
  else if (D <= 192) hipLaunchKernelGGL(head_norm_rope_kernel<3>, grid, block, 0, s, in, S, in_stride, col0, H, D, nr, out);
  else hipLaunchKernelGGL(head_norm_rope_kernel<4>, grid, block, 0, s, in, S, in_stride, col0, H, D, nr, out);
  return hipGetLastError();
}

}  // namespace mxa

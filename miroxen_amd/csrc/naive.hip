// Naive fp32 GPU attention: one 128-thread work-group per (query row, head).
// Behaviour of the reference's test oracle reference_kernel
// (src/kernels/attention.cu:292-348): fp32 dot products, expf, online
// max/sum over 128-key chunks, bf16 output, 0 when the row has no live key.
// Extended with the key-padding mask. Besides attn_reference it is the general
// path of flash_attn where the MFMA kernel's preconditions fail (operands not 2-byte
// aligned, masked Skv > 65536, K/V beyond 32-bit buffer offsets).
#include "attn_common.hpp"

namespace mxa {

namespace {

__device__ float block_reduce(float value, float* scratch, bool maximum) {
  __syncthreads();
  for (int off = 32; off; off >>= 1) {
    const float other = __shfl_xor(value, off);
    value = maximum ? fmaxf(value, other) : value + other;
  }
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = value;
  __syncthreads();
  return maximum ? fmaxf(scratch[0], scratch[1]) : scratch[0] + scratch[1];
}

__global__ void __launch_bounds__(128) naive_attn(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                                  uint16_t* o, mx_attn_params p) {
  __shared__ float weights[128], scratch[2];
  const int row = blockIdx.x, head = blockIdx.y, tid = threadIdx.x;
  const int kvh = head / (p.Hq / p.Hkv), D = p.D;
  int64_t end = p.Skv;
  if (p.causal) {
    const int64_t last = int64_t(p.q_offset) + row + 1;
    end = last < 0 ? 0 : (last < end ? last : end);
  }
  const uint16_t* qr = q + int64_t(row) * p.q_stride + int64_t(head) * D;
  float maximum = -__builtin_inff(), sum = 0.f, out = 0.f;
  for (int64_t start = 0; start < end; start += 128) {
    float score = -__builtin_inff();
    const int64_t key = start + tid;
    if (key < end && (!p.kv_valid || p.kv_valid[key])) {
      const uint16_t* kr = k + key * p.kv_stride + int64_t(kvh) * D;
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot = __builtin_fmaf(bf2f(qr[d]), bf2f(kr[d]), dot);
      score = dot * p.scale;
    }
    const float next = fmaxf(maximum, block_reduce(score, scratch, true));
    const float alpha = maximum == -__builtin_inff() ? 0.f : expf(maximum - next);
    const float w = score == -__builtin_inff() ? 0.f : expf(score - next);
    weights[tid] = w;
    const float tilesum = block_reduce(w, scratch, false);
    if (tid < D) {
      out *= alpha;
      for (int j = 0; j < 128 && start + j < end; ++j)
        out = __builtin_fmaf(weights[j], bf2f(v[(start + j) * p.kv_stride + int64_t(kvh) * D + tid]), out);
    }
    maximum = next;
    sum = sum * alpha + tilesum;
  }
  if (tid < D) o[int64_t(row) * p.o_stride + int64_t(head) * D + tid] = f2bf(sum > 0.f ? out / sum : 0.f);
}

}  // namespace

hipError_t launch_naive_attn(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                             const mx_attn_params& p, hipStream_t s) {
  hipLaunchKernelGGL(naive_attn, dim3(unsigned(p.Sq), unsigned(p.Hq)), dim3(128), 0, s, q, k, v, o, p);
  return hipGetLastError();
}

}  // namespace mxa

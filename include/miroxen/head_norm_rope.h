// Drop-in C++ face of mx_head_norm_rope for the reference's DiT blocks.
//
// Mirrors src/kernels/ops.h:30-41 of the reference (RopeMode and head_norm_rope:
// same names, argument order and meaning; cudaStream_t becomes hipStream_t).
// Errors surface as std::runtime_error, as the reference's MX_CHECK does.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "miroxen_attn.h"

namespace mx {

// Reference ops.h:35: INTERLEAVED pairs channels (2i, 2i+1) (Qwen-Image), HALF
// pairs (i, i + rot/2) (rotate_half; H3, Qwen3-VL); cos/sin are [S, rot/2].
enum RopeMode { ROPE_NONE = MX_ROPE_NONE, ROPE_INTERLEAVED = MX_ROPE_INTERLEAVED, ROPE_HALF = MX_ROPE_HALF };

// Reference ops.h:39-41: head h of token s is in[s*in_stride + col0 + h*D .. +D);
// per-head RMS-norm (skipped when norm_w is null), then RoPE of the first rot
// channels, written to out [S, H, D].
inline void head_norm_rope(const __hip_bfloat16* in, int64_t S, int64_t in_stride, int64_t col0, int H, int D,
                           const float* norm_w, float eps, const float* cos, const float* sin, int rot,
                           RopeMode mode, __hip_bfloat16* out, hipStream_t s) {
  if (mx_head_norm_rope(in, S, in_stride, col0, H, D, norm_w, eps, cos, sin, rot, int(mode), out, s) != MX_OK)
    throw std::runtime_error(std::string(mx_last_error()));
}

}  // namespace mx

// Drop-in C++ face of libmiroxen_attn.so for the reference's DiT blocks.
//
// Mirrors src/kernels/attention.h:12-39 of the reference: same namespace, struct,
// function names, argument order and meaning; cudaStream_t becomes hipStream_t.
// Errors surface as std::runtime_error, as the reference's MX_CHECK / MX_CUDA do
// (src/core/common.h:34-48). Everything forwards to the C ABI in miroxen_attn.h.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "miroxen_attn.h"

namespace mx {

using bf16 = __hip_bfloat16;

// Reference AttnParams (src/kernels/attention.h:12-18), plus the key-padding mask
// as a trailing, defaulted member: aggregate and field-by-field initialisation in
// existing callers keeps compiling.
struct AttnParams {
  int Sq = 0, Skv = 0, Hq = 0, Hkv = 0, D = 0;
  float scale = 0.f;  // 0 -> 1/sqrt(D)
  int causal = 0;
  int q_offset = 0;
  int64_t q_stride = 0, kv_stride = 0, o_stride = 0;
  const uint8_t* kv_valid = nullptr;  // optional device uint8[Skv], 0 = padded key
};

namespace detail {
inline mx_attn_params to_c(const AttnParams& p) {
  mx_attn_params c;
  c.Sq = p.Sq;
  c.Skv = p.Skv;
  c.Hq = p.Hq;
  c.Hkv = p.Hkv;
  c.D = p.D;
  c.scale = p.scale;
  c.causal = p.causal;
  c.q_offset = p.q_offset;
  c.q_stride = p.q_stride;
  c.kv_stride = p.kv_stride;
  c.o_stride = p.o_stride;
  c.kv_valid = p.kv_valid;
  return c;
}
inline void check(int rc) {
  if (rc != MX_OK) throw std::runtime_error(std::string(mx_last_error()));
}
}  // namespace detail

// Reference: flash_attn, src/kernels/attention.h:21-22.
inline void flash_attn(const bf16* q, const bf16* k, const bf16* v, bf16* o, const AttnParams& p, hipStream_t s) {
  const mx_attn_params c = detail::to_c(p);
  detail::check(mx_flash_attn(q, k, v, o, &c, s));
}

// Reference: flash_attn_fp8_workspace, src/kernels/attention.h:28.
inline size_t flash_attn_fp8_workspace(const AttnParams& p) {
  const mx_attn_params c = detail::to_c(p);
  return mx_flash_attn_fp8_workspace(&c);
}

// Reference: flash_attn_fp8_supported, src/kernels/attention.h:30.
inline bool flash_attn_fp8_supported(int device) {
  int out = 0;
  detail::check(mx_flash_attn_fp8_supported(device, &out));
  return out != 0;
}

// Reference: flash_attn_fp8_ok, src/kernels/attention.h:32.
inline bool flash_attn_fp8_ok(const bf16* q, const bf16* k, const bf16* v, const bf16* o, const AttnParams& p) {
  const mx_attn_params c = detail::to_c(p);
  int out = 0;
  detail::check(mx_flash_attn_fp8_ok(q, k, v, o, &c, &out));
  return out != 0;
}

// Reference: flash_attn_fp8, src/kernels/attention.h:33-34.
inline void flash_attn_fp8(const bf16* q, const bf16* k, const bf16* v, bf16* o, const AttnParams& p, void* ws,
                           hipStream_t s) {
  const mx_attn_params c = detail::to_c(p);
  detail::check(mx_flash_attn_fp8(q, k, v, o, &c, ws, s));
}

// Fused head_norm_rope(q), head_norm_rope(k) + flash_attn_fp8 (see mx_flash_attn_fp8_norm_rope):
// q/k are the raw projections; q_norm/k_norm may be null; throws when the shape is
// outside the quantized path (there is no fallback).
inline void flash_attn_fp8_norm_rope(const bf16* q, const bf16* k, const bf16* v, bf16* o, const AttnParams& p,
                                     const float* q_norm, const float* k_norm, float eps, const float* cos,
                                     const float* sin, int rot, int mode, void* ws, hipStream_t s) {
  const mx_attn_params c = detail::to_c(p);
  const mx_qk_norm_rope n{q_norm, k_norm, eps, cos, sin, rot, mode};
  detail::check(mx_flash_attn_fp8_norm_rope(q, k, v, o, &c, &n, ws, s));
}

// Reference: attn_reference, src/kernels/attention.h:37-38.
inline void attn_reference(const bf16* q, const bf16* k, const bf16* v, bf16* o, const AttnParams& p,
                           hipStream_t s) {
  const mx_attn_params c = detail::to_c(p);
  detail::check(mx_attn_reference(q, k, v, o, &c, s));
}

}  // namespace mx

// Drop-in C++ face of the block-scaled GEMM for the reference's DiT linears.
//
// Mirrors src/kernels/blockscale.h:12-37 of the reference (QMode, QMat, qmode_name,
// parse_qmode, qmode_supported, qdata_bytes, qscale_bytes, quantize_blockscaled,
// gemm_blockscaled: same names and argument order; cudaStream_t becomes hipStream_t,
// and gemm_blockscaled takes either the stream or, as the reference (blockscale.h:34),
// the caller's context: any object with a `stream` member convertible to hipStream_t,
// so `gemm_blockscaled(ctx, ...)` call sites compile unchanged; the kernel needs no
// cuBLASLt handle or workspace and runs on the current device). Errors surface as
// std::runtime_error, as the reference's MX_CHECK does.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>

#include "miroxen_attn.h"

namespace mx {

enum class QMode { BF16 = MX_QMODE_BF16, MXFP8 = MX_QMODE_MXFP8, NVFP4 = MX_QMODE_NVFP4 };

inline const char* qmode_name(QMode m) { return m == QMode::NVFP4 ? "fp4" : m == QMode::MXFP8 ? "fp8" : "bf16"; }

inline QMode parse_qmode(const std::string& s) {
  if (s == "fp4" || s == "nvfp4") return QMode::NVFP4;
  if (s == "fp8" || s == "mxfp8") return QMode::MXFP8;
  if (!(s == "bf16" || s.empty())) throw std::runtime_error("unknown compute precision " + s + " (use bf16 / fp8 / fp4)");
  return QMode::BF16;
}

namespace detail {
inline void bs_check(int rc) {
  if (rc != MX_OK) throw std::runtime_error(std::string(mx_last_error()));
}
}  // namespace detail

inline bool qmode_supported(QMode m, int device) {
  int ok = 0;
  detail::bs_check(mx_qmode_supported(int(m), device, &ok));
  return ok != 0;
}

struct QMat {
  void* q = nullptr;
  uint8_t* sf = nullptr;
  float* amax = nullptr;
};

inline size_t qdata_bytes(QMode m, int64_t rows, int64_t K) { return mx_qdata_bytes(int(m), rows, K); }
inline size_t qscale_bytes(QMode m, int64_t rows, int64_t K) { return mx_qscale_bytes(int(m), rows, K); }

inline void quantize_blockscaled(QMode m, const __hip_bfloat16* x, int64_t ldx, int64_t rows, int64_t K,
                                 const QMat& out, hipStream_t s) {
  detail::bs_check(mx_quantize_blockscaled(int(m), x, ldx, rows, K, out.q, out.sf, out.amax, s));
}

inline void gemm_blockscaled(hipStream_t s, QMode m, const QMat& W, const QMat& X, __hip_bfloat16* Y, int64_t ldy,
                             int64_t M, int64_t N, int64_t K, float beta = 0.f) {
  detail::bs_check(mx_gemm_blockscaled(int(m), W.q, W.sf, W.amax, X.q, X.sf, X.amax, Y, ldy, M, N, K, beta, s));
}

// The reference's signature (src/kernels/blockscale.h:34-35): the context's stream.
template <class Ctx, class = std::enable_if_t<std::is_convertible_v<decltype(std::declval<Ctx&>().stream), hipStream_t>>>
inline void gemm_blockscaled(Ctx& c, QMode m, const QMat& W, const QMat& X, __hip_bfloat16* Y, int64_t ldy,
                             int64_t M, int64_t N, int64_t K, float beta = 0.f) {
  gemm_blockscaled(static_cast<hipStream_t>(c.stream), m, W, X, Y, ldy, M, N, K, beta);
}

}  // namespace mx

// The reference's invalid-input checks (tests/attention_test.cu:178-208) through
// the C++ drop-in header: 11 bad parameter sets x {flash_attn, attn_reference}
// plus a null query must each throw std::runtime_error; the block-scaled GEMM
// header's sizes (the reference test's shapes, tests/blockscale_test.cpp:135-136)
// and its MX_CHECK-style rejections. Validation happens on the host before any
// launch, so this runs without a GPU.
#include <cstdio>
#include <limits>
#include <stdexcept>

#include "miroxen/attention.h"
#include "miroxen/blockscale.h"
#include "miroxen/head_norm_rope.h"

using namespace mx;

int main() {
  auto* b = reinterpret_cast<bf16*>(uintptr_t(256));  // never dereferenced: validation fails first
  AttnParams good;
  good.Sq = 1; good.Skv = 1; good.Hq = 1; good.Hkv = 1; good.D = 64;
  int rejected = 0;
  for (int i = 0; i < 11; ++i) {
    AttnParams p = good;
    switch (i) {
      case 0: p.Sq = 0; break;
      case 1: p.Skv = -1; break;
      case 2: p.Hq = 3; p.Hkv = 2; break;
      case 3: p.D = 80; break;
      case 4: p.causal = 2; break;
      case 5: p.Hkv = 0; break;
      case 6: p.q_stride = 63; break;
      case 7: p.kv_stride = -1; break;
      case 8: p.o_stride = 63; break;
      case 9: p.scale = std::numeric_limits<float>::quiet_NaN(); break;
      case 10: p.kv_stride = std::numeric_limits<int64_t>::max(); break;
    }
    for (auto fn : {flash_attn, attn_reference}) {
      try {
        fn(b, b, b, b, p, nullptr);
      } catch (const std::runtime_error&) {
        ++rejected;
      }
    }
  }
  try {
    flash_attn(nullptr, b, b, b, good, nullptr);
  } catch (const std::runtime_error& e) {
    ++rejected;
  }
  // head_norm_rope: the reference's MX_CHECK (ops.cu:201) rejects an odd D
  int nr_rejected = 0;
  try {
    head_norm_rope(b, 4, 256, 0, 2, 127, nullptr, 0.f, nullptr, nullptr, 0, ROPE_NONE, b, nullptr);
  } catch (const std::runtime_error&) {
    ++nr_rejected;
  }
  // block-scaled GEMM: sizes of the reference test's shapes, then host-side rejections
  int bs_ok = 0;
  bs_ok += qdata_bytes(QMode::MXFP8, 300, 1024) == size_t(300) * 1024;
  bs_ok += qscale_bytes(QMode::MXFP8, 300, 1024) == size_t(384) * 32;   // rows -> 384, K/32 = 32
  bs_ok += qscale_bytes(QMode::MXFP8, 129, 4160) == size_t(256) * 132;  // K/32 = 130 -> 132
  bs_ok += parse_qmode("fp8") == QMode::MXFP8 && parse_qmode("") == QMode::BF16 &&
           std::string(qmode_name(QMode::NVFP4)) == "fp4";
  QMat qm{b, reinterpret_cast<uint8_t*>(b), nullptr};
  auto* hb = reinterpret_cast<__hip_bfloat16*>(b);
  const auto throws = [](auto f) {
    try {
      f();
    } catch (const std::runtime_error&) {
      return 1;
    }
    return 0;
  };
  bs_ok += throws([&] { parse_qmode("int3"); });
  bs_ok += throws([&] { quantize_blockscaled(QMode::MXFP8, hb, 48, 4, 48, qm, nullptr); });  // K % 32
  bs_ok += throws([&] { quantize_blockscaled(QMode::BF16, hb, 64, 4, 64, qm, nullptr); });
  bs_ok += throws([&] { gemm_blockscaled(nullptr, QMode::MXFP8, qm, qm, hb, 64, 4, 64, 64, 0.5f); });  // beta
  bs_ok += throws([&] { gemm_blockscaled(nullptr, QMode::NVFP4, qm, qm, hb, 64, 4, 64, 64); });
  // the reference's call form: a context object carrying the stream (src/kernels/blockscale.h:34)
  struct RefCtx {
    int device = 0;
    hipStream_t stream = nullptr;
  } ctx;
  bs_ok += throws([&] { gemm_blockscaled(ctx, QMode::MXFP8, qm, qm, hb, 64, 4, 64, 64, 0.5f); });  // beta
  // the workspace query is pure host arithmetic
  AttnParams c2;
  c2.Sq = 4352; c2.Skv = 4352; c2.Hq = 24; c2.Hkv = 24; c2.D = 128;
  const size_t ws = flash_attn_fp8_workspace(c2);
  std::printf("invalid input checks: %d rejected; head_norm_rope %d rejected; blockscale %d/10 ok; "
              "config-2 workspace %zu bytes\n", rejected, nr_rejected, bs_ok, ws);
  return rejected == 23 && nr_rejected == 1 && bs_ok == 10 && ws > 0 ? 0 : 1;
}

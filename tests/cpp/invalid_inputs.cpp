// The reference's invalid-input checks (tests/attention_test.cu:178-208) through
// the C++ drop-in header: 11 bad parameter sets x {flash_attn, attn_reference}
// plus a null query must each throw std::runtime_error. Validation happens on the
// host before any launch, so this runs without a GPU.
#include <cstdio>
#include <limits>
#include <stdexcept>

#include "miroxen/attention.h"
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
  // the workspace query is pure host arithmetic
  AttnParams c2;
  c2.Sq = 4352; c2.Skv = 4352; c2.Hq = 24; c2.Hkv = 24; c2.D = 128;
  const size_t ws = flash_attn_fp8_workspace(c2);
  std::printf("invalid input checks: %d rejected; head_norm_rope %d rejected; config-2 workspace %zu bytes\n",
              rejected, nr_rejected, ws);
  return rejected == 23 && nr_rejected == 1 && ws > 0 ? 0 : 1;
}

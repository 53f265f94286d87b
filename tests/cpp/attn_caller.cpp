// A C++ caller of the drop-in header, as a DiT block of the reference would call it
// (src/models/qwen_image/dit.cpp through mx::flash_attn / mx::flash_attn_fp8): reads
// bf16 Q, K, V [S][H*D] and an optional uint8 key mask from <dir>, runs
//   mx::flash_attn                                   -> <dir>/o_bf16.bin
//   mx::flash_attn_fp8 with a caller workspace       -> <dir>/o_fp8.bin
// and prints flash_attn_fp8_ok and the workspace size. The test compares the outputs
// with the CPU oracle and with the same calls made through the Python binding.
// Usage: attn_caller <dir> <S> <H> <D> <masked 0|1>
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <vector>

#include "miroxen/attention.h"

static std::vector<char> read_file(const std::string& path, size_t bytes) {
  std::vector<char> b(bytes);
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f || std::fread(b.data(), 1, bytes, f) != bytes) throw std::runtime_error("cannot read " + path);
  std::fclose(f);
  return b;
}

static void write_file(const std::string& path, const void* p, size_t bytes) {
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f || std::fwrite(p, 1, bytes, f) != bytes) throw std::runtime_error("cannot write " + path);
  std::fclose(f);
}

#define HIP_OK(x)                                                                     \
  do {                                                                                \
    hipError_t e_ = (x);                                                              \
    if (e_ != hipSuccess) throw std::runtime_error(std::string(#x) + ": " + hipGetErrorString(e_)); \
  } while (0)

int main(int argc, char** argv) {
  if (argc != 6) {
    std::fprintf(stderr, "usage: %s <dir> <S> <H> <D> <masked>\n", argv[0]);
    return 2;
  }
  try {
    const std::string dir = argv[1];
    const int S = std::atoi(argv[2]), H = std::atoi(argv[3]), D = std::atoi(argv[4]);
    const bool masked = std::atoi(argv[5]) != 0;
    const size_t n = size_t(S) * H * D, bytes = n * 2;
    std::vector<char> hq = read_file(dir + "/q.bin", bytes), hk = read_file(dir + "/k.bin", bytes),
                      hv = read_file(dir + "/v.bin", bytes);
    mx::bf16 *q, *k, *v, *o;
    uint8_t* mask = nullptr;
    HIP_OK(hipMalloc(&q, bytes));
    HIP_OK(hipMalloc(&k, bytes));
    HIP_OK(hipMalloc(&v, bytes));
    HIP_OK(hipMalloc(&o, bytes));
    HIP_OK(hipMemcpy(q, hq.data(), bytes, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(k, hk.data(), bytes, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(v, hv.data(), bytes, hipMemcpyHostToDevice));
    if (masked) {
      std::vector<char> hm = read_file(dir + "/mask.bin", size_t(S));
      HIP_OK(hipMalloc(&mask, size_t(S)));
      HIP_OK(hipMemcpy(mask, hm.data(), size_t(S), hipMemcpyHostToDevice));
    }
    hipStream_t s;
    HIP_OK(hipStreamCreate(&s));

    mx::AttnParams p;  // the reference's field-by-field initialisation
    p.Sq = S;
    p.Skv = S;
    p.Hq = H;
    p.Hkv = H;
    p.D = D;
    p.kv_valid = mask;
    std::vector<char> out(bytes);

    mx::flash_attn(q, k, v, o, p, s);
    HIP_OK(hipStreamSynchronize(s));
    HIP_OK(hipMemcpy(out.data(), o, bytes, hipMemcpyDeviceToHost));
    write_file(dir + "/o_bf16.bin", out.data(), bytes);

    const size_t wsb = mx::flash_attn_fp8_workspace(p);
    void* ws = nullptr;
    HIP_OK(hipMalloc(&ws, wsb));
    const bool ok = mx::flash_attn_fp8_supported(0) && mx::flash_attn_fp8_ok(q, k, v, o, p);
    HIP_OK(hipMemset(o, 0, bytes));
    mx::flash_attn_fp8(q, k, v, o, p, ws, s);
    HIP_OK(hipStreamSynchronize(s));
    HIP_OK(hipMemcpy(out.data(), o, bytes, hipMemcpyDeviceToHost));
    write_file(dir + "/o_fp8.bin", out.data(), bytes);
    std::printf("fp8_ok %d workspace %zu\n", ok ? 1 : 0, wsb);

    HIP_OK(hipFree(ws));
    HIP_OK(hipFree(q));
    HIP_OK(hipFree(k));
    HIP_OK(hipFree(v));
    HIP_OK(hipFree(o));
    if (mask) HIP_OK(hipFree(mask));
    HIP_OK(hipStreamDestroy(s));
  } catch (const std::exception& e) {
    std::fprintf(stderr, "attn_caller: %s\n", e.what());
    return 1;
  }
  return 0;
}

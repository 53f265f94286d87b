// C-ABI entry points (declared in include/miroxen_attn.h). Host code only:
// argument validation, path selection and launches. Errors never cross the ABI
// as exceptions: every entry point returns a status and records a thread-local
// message (reference contract: MX_CHECK throws std::runtime_error,
// src/core/common.h:42-48; the C++ wrapper in include/miroxen/attention.h
// rethrows).
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <limits>
#include <mutex>

#include "attn_common.hpp"
#include "norm_rope.hpp"

namespace mxa {
hipError_t launch_head_norm_rope(const uint16_t*, int64_t, int64_t, int64_t, int, int, const NormRope&, uint16_t*,
                                 hipStream_t);
hipError_t launch_flash_bf16(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*,
                                  const mx_attn_params&, hipStream_t);
int flash_bf16_split_plan(const mx_attn_params&, int cus, int* full, int* units, int* parts);
hipError_t launch_naive_attn(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, const mx_attn_params&,
                             hipStream_t);
mx_sage_layout sage_layout(const mx_attn_params&);
hipError_t launch_sage_quantize(const uint16_t*, const uint16_t*, const uint16_t*, const mx_attn_params&, char*,
                                hipStream_t, const NormRope*, int q_group);
hipError_t launch_sage_attend(uint16_t*, const mx_attn_params&, const char*, hipStream_t);
void set_prologue_wait_ticks(uint64_t);
hipError_t launch_sage_fp8(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, const mx_attn_params&, char*,
                           hipStream_t);
size_t mx_qscale_size(int64_t rows, int64_t K);
hipError_t launch_mxfp8_quant(const uint16_t*, int64_t, int64_t, int64_t, uint8_t*, uint8_t*, hipStream_t);
hipError_t launch_mxfp8_gemm(const uint8_t*, const uint8_t*, const uint8_t*, const uint8_t*, uint16_t*, int64_t, int,
                             int, int, int, hipStream_t);
hipError_t launch_nvfp4_quant(const uint16_t*, int64_t, int64_t, int64_t, uint8_t*, uint8_t*, float*, hipStream_t);
hipError_t launch_nvfp4_gemm(const uint8_t*, const uint8_t*, const float*, const uint8_t*, const uint8_t*, const float*,
                             uint16_t*, int64_t, int, int, int, int, hipStream_t);
}  // namespace mxa

namespace {

// Masked calls keep one 64-bit liveness word per 64-key tile in LDS.
constexpr int64_t kMaxMaskedSkv = 1024 * 64;

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return MX_OK;
  return fail(MX_E_HIP, "%s: HIP %s", what, hipGetErrorString(e));
}

bool aligned(const void* x, uintptr_t a) { return (reinterpret_cast<uintptr_t>(x) & (a - 1)) == 0; }

// Reference validate(), src/kernels/attention.cu:350-369: same rules and order;
// fills dense strides and the default scale.
int validate(const void* q, const void* k, const void* v, const void* o, const mx_attn_params* in,
             mx_attn_params* out) {
  if (!in) return fail(MX_E_INVALID, "attention: null parameter block");
  mx_attn_params p = *in;
  if (!(p.Sq > 0 && p.Skv > 0 && p.Hq > 0 && p.Hkv > 0 && p.Hq % p.Hkv == 0))
    return fail(MX_E_INVALID, "attention: lengths/heads must be positive and Hq must be a multiple of Hkv");
  if (!(p.D == 64 || p.D == 72 || p.D == 128))
    return fail(MX_E_INVALID, "attention: unsupported head dimension %d", p.D);
  if (!(p.causal == 0 || p.causal == 1)) return fail(MX_E_INVALID, "attention: causal must be 0 or 1");
  if (!(q && k && v && o)) return fail(MX_E_INVALID, "attention: null tensor pointer");
  if (!std::isfinite(p.scale)) return fail(MX_E_INVALID, "attention: scale must be finite");
  const int64_t qdense = int64_t(p.Hq) * p.D, kdense = int64_t(p.Hkv) * p.D;
  if (!p.q_stride) p.q_stride = qdense;
  if (!p.kv_stride) p.kv_stride = kdense;
  if (!p.o_stride) p.o_stride = qdense;
  if (!(p.q_stride >= qdense && p.kv_stride >= kdense && p.o_stride >= qdense))
    return fail(MX_E_INVALID, "attention: token stride is smaller than a row");
  const int64_t limit = std::numeric_limits<int64_t>::max() / 2;
  if (!(p.q_stride <= limit / p.Sq && p.kv_stride <= limit / p.Skv && p.o_stride <= limit / p.Sq))
    return fail(MX_E_INVALID, "attention: tensor address range overflows");
  if (p.Hq > 65535) return fail(MX_E_INVALID, "attention: too many heads for the launch grid");
  if (p.scale == 0.f) p.scale = 1.f / std::sqrt(float(p.D));
  *out = p;
  return MX_OK;
}

// Reference with_defaults(), src/kernels/attention_fp8.cu:461-467.
mx_attn_params with_defaults(mx_attn_params p) {
  if (!p.q_stride) p.q_stride = int64_t(p.Hq) * p.D;
  if (!p.kv_stride) p.kv_stride = int64_t(p.Hkv) * p.D;
  if (!p.o_stride) p.o_stride = int64_t(p.Hq) * p.D;
  if (p.scale == 0.f && p.D > 0) p.scale = 1.f / std::sqrt(float(p.D));
  return p;
}

bool device_is_gfx950(int device) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return false;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
}

// Reference fp8_ok(), src/kernels/attention_fp8.cu:451-459: D == 64 or 128, no causal
// mask, aligned operands; for this build's kernels also a positive scale (the integer
// row max assumes a positive score scale), a quantized K/V head that 32-bit buffer
// offsets can address (skv_pad * D < 2^32), and a gfx950 device.
int fp8_ok(const void* q, const void* k, const void* v, const void* o, const mx_attn_params& p, bool* ok) {
  *ok = false;
  if (p.causal || (p.D != 128 && p.D != 64) || p.Sq <= 0 || p.Skv <= 0 || p.Hkv <= 0 || p.Hq <= 0 || p.Hq % p.Hkv) return MX_OK;
  // bf16 operands at their natural 2-byte alignment, any token stride: gfx950 serves the
  // kernels' 16-byte row loads and 4-byte stores at 2-byte granularity
  if (!aligned(q, 2) || !aligned(k, 2) || !aligned(v, 2) || !aligned(o, 2)) return MX_OK;
  if (!(p.scale > 0.f) || p.Hq > 65535 || (p.kv_valid && p.Skv > kMaxMaskedSkv)) return MX_OK;
  const int64_t skv_pad = (int64_t(p.Skv) + mxa::kKvPad - 1) / mxa::kKvPad * mxa::kKvPad;
  if (skv_pad * p.D >= (int64_t(1) << 32)) return MX_OK;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "flash_attn_fp8_ok");
  *ok = device_is_gfx950(dev);
  return MX_OK;
}

// The MFMA kernel's preconditions. Token strides need not be multiples of 8 (the
// reference's Aligned = false case, attention.cu:55-63, :383-389): the kernel's 16-byte
// K/V tile loads (buffer -> LDS), Q loads and 4-byte O stores are served at 2-byte
// granularity by gfx950's memory system, so one kernel covers both cases.
bool fast_bf16_ok(const void* q, const void* k, const void* v, const void* o, const mx_attn_params& p) {
  return aligned(q, 2) && aligned(k, 2) && aligned(v, 2) && aligned(o, 2) &&
         (!p.kv_valid || p.Skv <= kMaxMaskedSkv) &&
         int64_t(p.Skv) * p.kv_stride * 2 < (int64_t(1) << 32);  // K/V tiles read through 32-bit buffer offsets
}

// Fixed device scratch of mx_flash_attn_fp8_noalloc: the Sage workspace lives in this
// file-scope array (one copy per device, held until the process ends) instead of a
// caller allocation. Host code never passes the array's name to a kernel or a copy:
// on the host it is a stand-in symbol, and each device's copy is at its own address,
// looked up once per device with hipGetSymbolAddress (with that device current).
// Calls on one device are ordered through a per-device event (each call's stream
// waits for the previous call's last kernel), so calls on different streams do not
// overwrite each other's workspace; calls under stream capture skip the event (a
// graph cannot wait on work outside it), so a replay that overlaps another call on
// the device races on the scratch.
constexpr size_t kNoAllocScratchBytes = size_t(128) << 20;  // 128 MiB
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
struct ScratchDevice {
  std::once_flag once;
  hipError_t setup = hipSuccess;
  void* ptr = nullptr;
  hipEvent_t done = nullptr;
  std::mutex mu;
};
ScratchDevice g_scratch[kMaxDevices];

int scratch_of_current_device(ScratchDevice** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "flash_attn_fp8_noalloc");
  if (dev < 0 || dev >= kMaxDevices) return fail(MX_E_UNSUPPORTED, "flash_attn_fp8_noalloc: device %d", dev);
  ScratchDevice& S = g_scratch[dev];
  std::call_once(S.once, [&S] {
    void* ptr = nullptr;
    hipError_t r = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (r == hipSuccess && (!ptr || !aligned(ptr, 256))) r = hipErrorInvalidValue;
    if (r == hipSuccess) r = hipEventCreateWithFlags(&S.done, hipEventDisableTiming);
    if (r == hipSuccess) S.ptr = ptr;
    S.setup = r;
  });
  if (S.setup != hipSuccess) return hip_status(S.setup, "flash_attn_fp8_noalloc: scratch set-up");
  *out = &S;
  return MX_OK;
}

}  // namespace

extern "C" {

const char* mx_last_error(void) { return g_err; }

const char* mx_version(void) { return "miroxen_amd gfx950 bf16:pp8x32q-k64 sage:pipe4x32q-k64-d128,w8x32q-k64-d64-int8fp8"; }

int mx_flash_attn(const void* q, const void* k, const void* v, void* o, const mx_attn_params* p, void* stream) {
  mx_attn_params a;
  int rc = validate(q, k, v, o, p, &a);
  if (rc) return rc;
  auto s = static_cast<hipStream_t>(stream);
  auto qq = static_cast<const uint16_t*>(q);
  auto kk = static_cast<const uint16_t*>(k);
  auto vv = static_cast<const uint16_t*>(v);
  auto oo = static_cast<uint16_t*>(o);
  if (fast_bf16_ok(q, k, v, o, a)) return hip_status(mxa::launch_flash_bf16(qq, kk, vv, oo, a, s), "flash_attn");
  return hip_status(mxa::launch_naive_attn(qq, kk, vv, oo, a, s), "flash_attn");
}

int mx_flash_attn_uses_mfma(const void* q, const void* k, const void* v, const void* o, const mx_attn_params* p,
                            int* mfma) {
  if (!mfma) return fail(MX_E_INVALID, "flash_attn_uses_mfma: null output");
  mx_attn_params a;
  int rc = validate(q, k, v, o, p, &a);
  if (rc) return rc;
  *mfma = fast_bf16_ok(q, k, v, o, a) ? 1 : 0;
  return MX_OK;
}

int mx_flash_attn_split_plan(const mx_attn_params* p, int cus, int* full, int* units, int* parts) {
  if (!p || !full || !units || !parts) return fail(MX_E_INVALID, "flash_attn_split_plan: null argument");
  if (p->Sq <= 0 || p->Skv <= 0 || p->Hq <= 0) return fail(MX_E_INVALID, "flash_attn_split_plan: empty shape");
  if (cus <= 0) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_status(e, "flash_attn_split_plan");
  }
  mxa::flash_bf16_split_plan(*p, cus, full, units, parts);
  return MX_OK;
}

int mx_attn_reference(const void* q, const void* k, const void* v, void* o, const mx_attn_params* p, void* stream) {
  mx_attn_params a;
  int rc = validate(q, k, v, o, p, &a);
  if (rc) return rc;
  return hip_status(mxa::launch_naive_attn(static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                                           static_cast<const uint16_t*>(v), static_cast<uint16_t*>(o), a,
                                           static_cast<hipStream_t>(stream)),
                    "attn_reference");
}

size_t mx_flash_attn_fp8_workspace(const mx_attn_params* p) {
  if (!p || p->Sq <= 0 || p->Skv <= 0 || p->D <= 0 || p->Hq <= 0 || p->Hkv <= 0) return 0;
  return mxa::sage_layout(*p).total;
}

int mx_sage_layout_of(const mx_attn_params* p, mx_sage_layout* out) {
  if (!p || !out) return fail(MX_E_INVALID, "sage_layout: null argument");
  if (p->Sq <= 0 || p->Skv <= 0 || p->D <= 0 || p->Hq <= 0 || p->Hkv <= 0)
    return fail(MX_E_INVALID, "sage_layout: empty shape");
  *out = mxa::sage_layout(*p);
  return MX_OK;
}

int mx_flash_attn_fp8_supported(int device, int* supported) {
  if (!supported) return fail(MX_E_INVALID, "flash_attn_fp8_supported: null output");
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess) return hip_status(e, "flash_attn_fp8_supported");
  if (device < 0 || device >= count) return fail(MX_E_INVALID, "flash_attn_fp8_supported: no device %d", device);
  *supported = device_is_gfx950(device) ? 1 : 0;
  return MX_OK;
}

int mx_flash_attn_fp8_ok(const void* q, const void* k, const void* v, const void* o, const mx_attn_params* p,
                         int* ok) {
  if (!p || !ok) return fail(MX_E_INVALID, "flash_attn_fp8_ok: null argument");
  bool b = false;
  int rc = fp8_ok(q, k, v, o, with_defaults(*p), &b);
  *ok = b ? 1 : 0;
  return rc;
}

// Validation shared by the quantized entry points: the reference validate()
// rules, then the fp8_ok() conditions, then the workspace contract.
static int sage_args(const void* q, const void* k, const void* v, const void* o, const mx_attn_params* p,
                     const void* ws, mx_attn_params* a, bool* ok) {
  int rc = validate(q, k, v, o, p, a);
  if (rc) return rc;
  rc = fp8_ok(q, k, v, o, *a, ok);
  if (rc || !*ok || !ws) return rc;
  if (!aligned(ws, 256)) return fail(MX_E_INVALID, "flash_attn_fp8: workspace must be 256-byte aligned");
  return MX_OK;
}

int mx_flash_attn_fp8(const void* q, const void* k, const void* v, void* o, const mx_attn_params* p, void* ws,
                      void* stream) {
  mx_attn_params a;
  bool ok = false;
  int rc = sage_args(q, k, v, o, p, ws, &a, &ok);
  if (rc) return rc;
  if (!ws || !ok) return mx_flash_attn(q, k, v, o, p, stream);  // reference :491
  return hip_status(mxa::launch_sage_fp8(static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                                         static_cast<const uint16_t*>(v), static_cast<uint16_t*>(o), a,
                                         static_cast<char*>(ws), static_cast<hipStream_t>(stream)),
                    "flash_attn_fp8");
}

int mx_flash_attn_fp8_noalloc(const void* q, const void* k, const void* v, void* o, const mx_attn_params* p,
                              void* stream) {
  mx_attn_params a;
  int rc = validate(q, k, v, o, p, &a);
  if (rc) return rc;
  bool ok = false;
  rc = fp8_ok(q, k, v, o, a, &ok);
  if (rc) return rc;
  if (!ok) return mx_flash_attn(q, k, v, o, p, stream);  // as mx_flash_attn_fp8: no workspace needed
  const size_t need = mxa::sage_layout(a).total;
  if (need > kNoAllocScratchBytes)
    return fail(MX_E_UNSUPPORTED, "flash_attn_fp8_noalloc: workspace of %zu bytes exceeds the %zu-byte scratch",
                need, kNoAllocScratchBytes);
  ScratchDevice* S = nullptr;
  rc = scratch_of_current_device(&S);
  if (rc) return rc;
  auto st = static_cast<hipStream_t>(stream);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(st, &cap);
  if (e != hipSuccess) return hip_status(e, "flash_attn_fp8_noalloc");
  const bool ordered = cap == hipStreamCaptureStatusNone;
  std::unique_lock<std::mutex> lock(S->mu, std::defer_lock);
  if (ordered) {
    lock.lock();
    e = hipStreamWaitEvent(st, S->done, 0);
    if (e != hipSuccess) return hip_status(e, "flash_attn_fp8_noalloc");
  }
  // the prologue rewrites every region the attention kernel reads and zeroes the
  // split arrival counters, so nothing is left over from the previous call
  e = mxa::launch_sage_fp8(static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                           static_cast<const uint16_t*>(v), static_cast<uint16_t*>(o), a,
                           static_cast<char*>(S->ptr), st);
  if (e == hipSuccess && ordered) e = hipEventRecord(S->done, st);
  return hip_status(e, "flash_attn_fp8_noalloc");
}

int mx_sage_quantize(const void* q, const void* k, const void* v, const mx_attn_params* p, void* ws,
                     void* stream) {
  mx_attn_params a;
  bool ok = false;
  int rc = sage_args(q, k, v, q, p, ws, &a, &ok);
  if (rc) return rc;
  if (!ok) return fail(MX_E_UNSUPPORTED, "sage_quantize: arguments not supported by the quantized path");
  if (!ws) return fail(MX_E_INVALID, "sage_quantize: null workspace");
  return hip_status(mxa::launch_sage_quantize(static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                                              static_cast<const uint16_t*>(v), a, static_cast<char*>(ws),
                                              static_cast<hipStream_t>(stream), nullptr, 16),
                    "sage_quantize");
}

int mx_sage_prologue_wait_ticks(int64_t ticks) {
  if (ticks < 0) return fail(MX_E_INVALID, "sage_prologue_wait_ticks: negative bound");
  mxa::set_prologue_wait_ticks(uint64_t(ticks));
  return MX_OK;
}

int mx_sage_quantize_qgroup(const void* q, const void* k, const void* v, const mx_attn_params* p, void* ws,
                            int q_group, void* stream) {
  if (q_group != 16 && q_group != 64) return fail(MX_E_INVALID, "sage_quantize_qgroup: q_group must be 16 or 64");
  mx_attn_params a;
  bool ok = false;
  int rc = sage_args(q, k, v, q, p, ws, &a, &ok);
  if (rc) return rc;
  if (!ok) return fail(MX_E_UNSUPPORTED, "sage_quantize_qgroup: arguments not supported by the quantized path");
  if (!ws) return fail(MX_E_INVALID, "sage_quantize_qgroup: null workspace");
  return hip_status(mxa::launch_sage_quantize(static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                                              static_cast<const uint16_t*>(v), a, static_cast<char*>(ws),
                                              static_cast<hipStream_t>(stream), nullptr, q_group),
                    "sage_quantize_qgroup");
}

// Fused head_norm_rope + Sage prologue: the head_norm_rope rules (reference
// ops.cu:201) for the norm/rope block, the quantized path's rules for the rest.
static int norm_rope_args(const mx_qk_norm_rope* nr, const mx_attn_params& a, const char* who,
                          mxa::NormRope out[2]) {
  if (!nr) return fail(MX_E_INVALID, "%s: null norm/rope block", who);
  if (a.D != 128) return fail(MX_E_UNSUPPORTED, "%s: the fused norm/rope prologue is built for D = 128", who);
  const int rot = nr->rot, mode = nr->mode;
  if (!(rot >= 0 && rot <= a.D && rot % 2 == 0)) return fail(MX_E_INVALID, "%s: D=%d rot=%d", who, a.D, rot);
  if (!(mode == MX_ROPE_NONE || mode == MX_ROPE_INTERLEAVED || mode == MX_ROPE_HALF))
    return fail(MX_E_INVALID, "%s: unknown rope mode %d", who, mode);
  if (mode != MX_ROPE_NONE && rot > 0 && (!nr->cos || !nr->sin))
    return fail(MX_E_INVALID, "%s: rope needs cos and sin tables", who);
  out[0] = mxa::NormRope{nr->q_norm, nr->eps, nr->cos, nr->sin, rot, mode};
  out[1] = mxa::NormRope{nr->k_norm, nr->eps, nr->cos, nr->sin, rot, mode};
  const int64_t rows = a.Sq > a.Skv ? a.Sq : a.Skv;
  if (!mxa::nr128_supported(out[0], rows) || !mxa::nr128_supported(out[1], rows))
    return fail(MX_E_UNSUPPORTED,
                "%s: needs 16-byte aligned norm weights and rope tables, rot %% 8 == 0 (rotate-half: %% 16)", who);
  return MX_OK;
}

int mx_sage_quantize_norm_rope(const void* q, const void* k, const void* v, const mx_attn_params* p,
                               const mx_qk_norm_rope* nr, void* ws, void* stream) {
  mx_attn_params a;
  bool ok = false;
  int rc = sage_args(q, k, v, q, p, ws, &a, &ok);
  if (rc) return rc;
  if (!ok) return fail(MX_E_UNSUPPORTED, "sage_quantize_norm_rope: arguments not supported by the quantized path");
  if (!ws) return fail(MX_E_INVALID, "sage_quantize_norm_rope: null workspace");
  mxa::NormRope n[2];
  rc = norm_rope_args(nr, a, "sage_quantize_norm_rope", n);
  if (rc) return rc;
  return hip_status(mxa::launch_sage_quantize(static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                                              static_cast<const uint16_t*>(v), a, static_cast<char*>(ws),
                                              static_cast<hipStream_t>(stream), n, 16),
                    "sage_quantize_norm_rope");
}

int mx_flash_attn_fp8_norm_rope(const void* q, const void* k, const void* v, void* o, const mx_attn_params* p,
                                const mx_qk_norm_rope* nr, void* ws, void* stream) {
  mx_attn_params a;
  bool ok = false;
  int rc = sage_args(q, k, v, o, p, ws, &a, &ok);
  if (rc) return rc;
  if (!ok) return fail(MX_E_UNSUPPORTED, "flash_attn_fp8_norm_rope: arguments not supported by the quantized path");
  if (!ws) return fail(MX_E_INVALID, "flash_attn_fp8_norm_rope: null workspace");
  mxa::NormRope n[2];
  rc = norm_rope_args(nr, a, "flash_attn_fp8_norm_rope", n);
  if (rc) return rc;
  auto s = static_cast<hipStream_t>(stream);
  rc = hip_status(mxa::launch_sage_quantize(static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                                            static_cast<const uint16_t*>(v), a, static_cast<char*>(ws), s, n, 16),
                  "flash_attn_fp8_norm_rope prologue");
  if (rc) return rc;
  return hip_status(mxa::launch_sage_attend(static_cast<uint16_t*>(o), a, static_cast<const char*>(ws), s),
                    "flash_attn_fp8_norm_rope");
}

int mx_sage_attend(void* o, const mx_attn_params* p, const void* ws, void* stream) {
  if (!p) return fail(MX_E_INVALID, "sage_attend: null parameter block");
  if (!o || !ws) return fail(MX_E_INVALID, "sage_attend: null pointer");
  mx_attn_params a;
  // q/k/v are not read by the main kernel; the workspace stands in for them.
  bool ok = false;
  int rc = sage_args(ws, ws, ws, o, p, ws, &a, &ok);
  if (rc) return rc;
  if (!ok) return fail(MX_E_UNSUPPORTED, "sage_attend: arguments not supported by the quantized path");
  return hip_status(mxa::launch_sage_attend(static_cast<uint16_t*>(o), a, static_cast<const char*>(ws),
                                            static_cast<hipStream_t>(stream)),
                    "sage_attend");
}

int mx_head_norm_rope(const void* in, int64_t S, int64_t in_stride, int64_t col0, int H, int D, const float* norm_w,
                      float eps, const float* cos, const float* sin, int rot, int mode, void* out, void* stream) {
  if (S <= 0) return MX_OK;  // reference ops.cu:200
  // reference MX_CHECK, ops.cu:201
  if (!(D % 2 == 0 && D > 0 && D <= 256 && rot >= 0 && rot <= D && rot % 2 == 0))
    return fail(MX_E_INVALID, "head_norm_rope: D=%d rot=%d", D, rot);
  if (!(mode == MX_ROPE_NONE || mode == MX_ROPE_INTERLEAVED || mode == MX_ROPE_HALF))
    return fail(MX_E_INVALID, "head_norm_rope: unknown rope mode %d", mode);
  if (!in || !out || H <= 0 || in_stride < col0 + int64_t(H) * D || col0 < 0)
    return fail(MX_E_INVALID, "head_norm_rope: bad tensor arguments");
  if (mode != MX_ROPE_NONE && rot > 0 && (!cos || !sin))
    return fail(MX_E_INVALID, "head_norm_rope: rope needs cos and sin tables");
  const mxa::NormRope nr{norm_w, eps, cos, sin, rot, mode};
  return hip_status(mxa::launch_head_norm_rope(static_cast<const uint16_t*>(in), S, in_stride, col0, H, D, nr,
                                               static_cast<uint16_t*>(out), static_cast<hipStream_t>(stream)),
                    "head_norm_rope");
}

int mx_qmode_supported(int mode, int device, int* supported) {
  if (!supported) return fail(MX_E_INVALID, "qmode_supported: null output");
  if (mode != MX_QMODE_BF16 && mode != MX_QMODE_MXFP8 && mode != MX_QMODE_NVFP4)
    return fail(MX_E_INVALID, "qmode_supported: unknown mode %d", mode);
  if (mode == MX_QMODE_BF16) return *supported = 1, MX_OK;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess) return hip_status(e, "qmode_supported");
  if (device < 0 || device >= count) return fail(MX_E_INVALID, "qmode_supported: no device %d", device);
  *supported = device_is_gfx950(device) ? 1 : 0;  // MXFP8 and NVFP4
  return MX_OK;
}

size_t mx_qdata_bytes(int mode, int64_t rows, int64_t K) {
  if (rows <= 0 || K <= 0) return 0;
  return size_t(rows) * size_t(K) / (mode == MX_QMODE_NVFP4 ? 2 : 1);
}

size_t mx_qscale_bytes(int mode, int64_t rows, int64_t K) {
  if (rows <= 0 || K <= 0) return 0;
  const int64_t vec = mode == MX_QMODE_NVFP4 ? 16 : 32;
  return size_t((rows + 127) / 128 * 128) * size_t((K / vec + 3) / 4 * 4);
}

int mx_quantize_blockscaled(int mode, const void* x, int64_t ldx, int64_t rows, int64_t K, void* q, void* sf,
                            float* amax, void* stream) {
  if (mode == MX_QMODE_BF16) return fail(MX_E_INVALID, "quantize_blockscaled: bf16 is not a quantized mode");
  if (mode != MX_QMODE_MXFP8 && mode != MX_QMODE_NVFP4)
    return fail(MX_E_INVALID, "quantize_blockscaled: unknown mode %d", mode);
  // reference MX_CHECK, blockscale.cu:116
  if (!(K % 32 == 0 && ldx % 8 == 0 && aligned(x, 16)))
    return fail(MX_E_INVALID, "quantize_blockscaled: need K%%32==0, ldx%%8==0, 16B-aligned input");
  if (rows == 0) return MX_OK;
  if (rows < 0 || K <= 0 || ldx < K || !x || !q || !sf || !aligned(q, mode == MX_QMODE_NVFP4 ? 8 : 16))
    return fail(MX_E_INVALID, "quantize_blockscaled: bad tensor arguments");
  if (mode == MX_QMODE_NVFP4) {
    if (!amax || !aligned(amax, 4)) return fail(MX_E_INVALID, "quantize_blockscaled: NVFP4 needs the amax pointer");
    return hip_status(mxa::launch_nvfp4_quant(static_cast<const uint16_t*>(x), ldx, rows, K, static_cast<uint8_t*>(q),
                                              static_cast<uint8_t*>(sf), amax, static_cast<hipStream_t>(stream)),
                      "quantize_blockscaled");
  }
  return hip_status(mxa::launch_mxfp8_quant(static_cast<const uint16_t*>(x), ldx, rows, K, static_cast<uint8_t*>(q),
                                            static_cast<uint8_t*>(sf), static_cast<hipStream_t>(stream)),
                    "quantize_blockscaled");
}

int mx_gemm_blockscaled(int mode, const void* wq, const void* wsf, const float* wamax, const void* xq, const void* xsf,
                        const float* xamax, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, float beta,
                        void* stream) {
  if (M == 0 || N == 0) return MX_OK;  // reference :136
  if (!(beta == 0.f || beta == 1.f)) return fail(MX_E_INVALID, "gemm_blockscaled: beta must be 0 or 1");
  if (mode != MX_QMODE_MXFP8 && mode != MX_QMODE_NVFP4)
    return fail(MX_E_INVALID, "gemm_blockscaled: %s", mode == MX_QMODE_BF16 ? "bf16 is not a quantized mode"
                                                                           : "unknown mode");
  if (mode == MX_QMODE_NVFP4 && (!wamax || !xamax || !aligned(wamax, 4) || !aligned(xamax, 4)))
    return fail(MX_E_INVALID, "gemm_blockscaled: NVFP4 needs both amax pointers");
  if (M < 0 || N < 0 || K <= 0 || K % 32 || ldy < N || !wq || !wsf || !xq || !xsf || !y || !aligned(wq, 16) ||
      !aligned(xq, 16) || !aligned(wsf, 4) || !aligned(xsf, 4) || !aligned(y, 2))
    return fail(MX_E_INVALID, "gemm_blockscaled: bad arguments (M=%lld N=%lld K=%lld)", (long long)M, (long long)N,
                (long long)K);
  // 32-bit buffer offsets within a 256-row tile's operand, and int grid coordinates
  if ((N + 255) / 256 * 256 * K >= (int64_t(1) << 31) || (M + 255) / 256 * 256 * K >= (int64_t(1) << 31) ||
      M > 0x7fffffff || N > 0x7fffffff)
    return fail(MX_E_UNSUPPORTED, "gemm_blockscaled: matrix too large for 32-bit offsets");
  if (mode == MX_QMODE_NVFP4)
    return hip_status(mxa::launch_nvfp4_gemm(static_cast<const uint8_t*>(wq), static_cast<const uint8_t*>(wsf), wamax,
                                             static_cast<const uint8_t*>(xq), static_cast<const uint8_t*>(xsf), xamax,
                                             static_cast<uint16_t*>(y), ldy, int(M), int(N), int(K),
                                             beta == 1.f ? 1 : 0, static_cast<hipStream_t>(stream)),
                      "gemm_blockscaled");
  return hip_status(mxa::launch_mxfp8_gemm(static_cast<const uint8_t*>(wq), static_cast<const uint8_t*>(wsf),
                                           static_cast<const uint8_t*>(xq), static_cast<const uint8_t*>(xsf),
                                           static_cast<uint16_t*>(y), ldy, int(M), int(N), int(K), beta == 1.f ? 1 : 0,
                                           static_cast<hipStream_t>(stream)),
                    "gemm_blockscaled");
}

}  // extern "C"

/*
 * miroxen_attn.h — C ABI of the MI355X (gfx950) DiT joint-attention library
 * (libmiroxen_attn.so). Plain pointers, sizes and a hipStream_t passed as void*;
 * no C++ or torch types. Every entry point returns 0 on success or a negative
 * MX_E* code; mx_last_error() returns the message of the calling thread's last
 * failure (thread-local, valid until that thread's next call).
 *
 * Tensor layouts follow the reference (src/kernels/attention.h:6-10):
 *   q: [Sq, Hq, D], k/v: [Skv, Hkv, D], o: [Sq, Hq, D], bf16, token-major;
 *   *_stride = elements between adjacent tokens (0 = dense H*D).
 * All calls are stream-ordered and asynchronous (no host synchronisation) and
 * run on the calling thread's current HIP device. The library allocates no
 * device memory: the Sage path works in a caller-provided workspace.
 */
#ifndef MIROXEN_ATTN_H
#define MIROXEN_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MX_OK = 0,
  MX_E_INVALID = -1, /* argument rejected (reference: MX_CHECK -> std::runtime_error) */
  MX_E_HIP = -2,     /* HIP runtime / launch error (reference: MX_CUDA / MX_KCHECK) */
  MX_E_UNSUPPORTED = -3
};

/* Reference: struct AttnParams, src/kernels/attention.h:12-18. Same fields in the
 * same order; kv_valid is new (key-padding mask) and sits last, so callers that
 * zero-initialise the struct and set fields one by one keep working.
 *   scale == 0 -> 1/sqrt(D); causal: query i sees keys [0, q_offset + i].
 *   kv_valid: optional device pointer to uint8 [Skv], 0 = padded key (score -inf),
 *   shared by all heads; NULL = every key valid. */
typedef struct mx_attn_params {
  int Sq, Skv, Hq, Hkv, D;
  float scale;
  int causal;
  int q_offset;
  int64_t q_stride, kv_stride, o_stride;
  const uint8_t* kv_valid;
} mx_attn_params;

/* Reference: mx::flash_attn, src/kernels/attention.h:21-22 (impl attention.cu:409-417).
 * D in {64,72,128}; bf16 in, fp32 accumulate, bf16 out. Invalid arguments ->
 * MX_E_INVALID with the reference's validate() rules (attention.cu:350-369).
 * Stream-ordered, no allocation, no host sync. Grids of few units (the last round
 * leaves most CUs idle, see mx_flash_attn_split_plan) run split into key ranges whose
 * partials live in a fixed library-owned device region (16 MiB per device); such
 * calls on one device are ordered by an event, calls that do not split share nothing.
 * UNDER STREAM CAPTURE a call never splits, so a captured replay of a shape that
 * splits eagerly gives a result that differs from the eager one by rounding (the
 * merge stores fp16 partials); both meet the BF16 tolerance. */
int mx_flash_attn(const void* q, const void* k, const void* v, void* o, const mx_attn_params* p,
                  void* stream);

/* Reference: mx::flash_attn_fp8_workspace, src/kernels/attention.h:28 (attention_fp8.cu:471-473).
 * Bytes of workspace flash_attn_fp8 needs (0 if the shape is empty). */
size_t mx_flash_attn_fp8_workspace(const mx_attn_params* p);

/* Reference: mx::flash_attn_fp8_supported, src/kernels/attention.h:30 (attention_fp8.cu:475-482).
 * *supported = 1 when `device` is a gfx950 (INT8 + OCP-FP8 MFMA). */
int mx_flash_attn_fp8_supported(int device, int* supported);

/* Reference: mx::flash_attn_fp8_ok, src/kernels/attention.h:32 (attention_fp8.cu:451-459, 484-486).
 * *ok = 1 when flash_attn_fp8 would take the quantized path for these arguments. */
int mx_flash_attn_fp8_ok(const void* q, const void* k, const void* v, const void* o,
                         const mx_attn_params* p, int* ok);

/* Reference: mx::flash_attn_fp8, src/kernels/attention.h:33-34 (attention_fp8.cu:488-500).
 * Sage attention: Q/K -> INT8 (Q per 16 tokens, K per 64 tokens after subtracting
 * the per-channel K mean), V -> OCP e4m3 per channel, INT8 QK^T and FP8 PV MFMA,
 * fp32 accumulation. ws: >= mx_flash_attn_fp8_workspace(p) bytes, 256-byte aligned.
 * Falls back to mx_flash_attn when ws == NULL or flash_attn_fp8_ok is false.
 * o may alias q (at D = 128 the attention kernel reads each unit's Q rows before any
 * of that unit's output is written; otherwise it reads only the workspace). */
int mx_flash_attn_fp8(const void* q, const void* k, const void* v, void* o, const mx_attn_params* p,
                      void* ws, void* stream);

/* No counterpart in the reference (a diagnostic query): *mfma = 1 when mx_flash_attn
 * runs the MFMA kernel for these arguments, 0 when it runs the general (naive) kernel.
 * Validates like mx_flash_attn; launches nothing. */
int mx_flash_attn_uses_mfma(const void* q, const void* k, const void* v, const void* o, const mx_attn_params* p,
                            int* mfma);

/* No counterpart in the reference (a diagnostic query): how mx_flash_attn splits the
 * work of these parameters on a device with `cus` compute units (cus <= 0: the current
 * device). The first *full units (head, 256-query tile) run whole; each of the last
 * *units units runs as *parts key ranges whose partial outputs a merge kernel combines
 * (parts == 1: no split). A split call keeps its partials in a fixed 16 MiB device
 * region (one per device, calls ordered by an event); only splits whose partials fit it
 * are planned. Causal calls and calls under stream capture run unsplit. Launches
 * nothing. */
int mx_flash_attn_split_plan(const mx_attn_params* p, int cus, int* full, int* units, int* parts);

/* No counterpart in the reference. For callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc):
 * mx_flash_attn_fp8 with the workspace taken from a fixed library-owned device scratch
 * of 128 MiB (one per device, held until the process ends) instead of an argument.
 * Allocates nothing. Shapes whose workspace (mx_flash_attn_fp8_workspace) exceeds the
 * scratch return MX_E_UNSUPPORTED; arguments the quantized path does not take fall
 * back to mx_flash_attn, as in mx_flash_attn_fp8 (which allocates nothing either).
 * Every call on a device shares that device's scratch; eager calls are ordered by a
 * per-device event (a call on another stream or host thread waits on the device for
 * the previous call to finish). Calls under stream capture skip that event: a graph
 * replay that overlaps another call on the same device races on the scratch, and the
 * caller must serialise them. */
int mx_flash_attn_fp8_noalloc(const void* q, const void* k, const void* v, void* o, const mx_attn_params* p,
                              void* stream);

/* Reference: mx::attn_reference, src/kernels/attention.h:37-38 (attention.cu:313-348, 419-423).
 * Slow naive GPU attention (fp32 softmax), for tests only. */
int mx_attn_reference(const void* q, const void* k, const void* v, void* o, const mx_attn_params* p,
                      void* stream);

/* ---- Sage pieces, exposed for bit-exact parity tests and split timing ----
 * No single reference counterpart: these are the two halves of
 * flash_attn_fp8's run<D>() (src/kernels/attention_fp8.cu:422-449). */

/* Byte offsets of the workspace regions (256-byte aligned each) and padded lengths.
 *   qi [Hq][sq_pad][D] int8, ki [Hkv][skv_pad][D] int8, vt [Hkv][D][skv_pad] e4m3,
 *   qs [Hq][sq_pad/16] f32, ks [Hkv][skv_pad/64] f32, km [Hkv][D] f32 (K mean),
 *   va [Hkv][D] f32 (V abs-max), part: kv_stats partials, tab (after part): per key
 *   tile its 64 liveness bits and K scale, for the attention kernel,
 *   split: partial outputs of the key-range-split work-groups that balance the
 *   attention grid's last round over an MI355X's 256 CUs (split_units units of
 *   split_qt query rows in split_parts parts each; 0 when the grid divides evenly),
 *   cnt: one int32 arrival counter per split unit (zeroed by the prologue, left zero
 *   by the kernel). Every field is a pure function of the parameters (no device
 *   query), as the reference's layout (src/kernels/attention_fp8.cu:471-473). */
typedef struct mx_sage_layout {
  int64_t sq_pad, skv_pad;
  size_t qi, ki, vt, qs, ks, km, va, part, split, cnt, total;
  int split_units, split_parts;
  int split_qt; /* query rows per grid unit of the attention kernel (128 or 256) */
  size_t tab;   /* [Hkv][skv_pad/64 + 1] 16-byte tile entries: liveness bits, K scale (negated
                   when some key of the tile is dead) */
  size_t flg;   /* [Hkv][nb] 64-bit ready flags of the one-pass K/V prologue, one per
                   256-token statistics block (nb = ceil(Skv/256)) */
} mx_sage_layout;
int mx_sage_layout_of(const mx_attn_params* p, mx_sage_layout* out);

/* Prologue only: kv_stats, Q/K INT8 quantization, V e4m3 quantization into ws. */
int mx_sage_quantize(const void* q, const void* k, const void* v, const mx_attn_params* p, void* ws,
                     void* stream);

/* mx_sage_quantize with a choice of Q scale group: q_group 16 is the reference's
 * (one Q scale per 16 tokens, attention_fp8.cu:435-438); 64 gives one Q scale per
 * 64-token block, the grouping the config-3 workload specifies. No reference
 * counterpart. The workspace layout is unchanged (a 64-token scale is stored in each
 * of its four 16-token entries), so mx_sage_attend runs on it as it is. */
int mx_sage_quantize_qgroup(const void* q, const void* k, const void* v, const mx_attn_params* p, void* ws,
                            int q_group, void* stream);

/* Test hook, no reference counterpart: the bound, in ticks of the 100 MHz chip clock
 * (default 20000 = 200 us), on how long a work-group of the one-pass K/V prologue waits
 * for the other statistics blocks of its head before it computes their partials from K
 * and V itself (same bytes, so the workspace does not change). 0 = one look. Process-wide;
 * for tests of that recompute path. */
int mx_sage_prologue_wait_ticks(int64_t ticks);

/* Main kernel only, on a workspace already filled by mx_sage_quantize (or
 * mx_sage_quantize_qgroup / mx_sage_quantize_norm_rope). A workspace last used by
 * mx_flash_attn_fp8 is not enough: at D = 128 that call quantizes Q inside its attention
 * kernel and leaves the workspace's Q regions unwritten. */
int mx_sage_attend(void* o, const mx_attn_params* p, const void* ws, void* stream);

/* Message of this thread's last failed call ("" if none). */
const char* mx_last_error(void);

/* Library build identifier (kernel variant string). */
const char* mx_version(void);

/* Reference: mx::head_norm_rope, src/kernels/ops.h:37-41 (impl ops.cu:87-119, :197-210),
 * the step that feeds attention in every DiT block: for each token s < S and head
 * h < H, x = in[s*in_stride + col0 + h*D .. +D) (bf16); if norm_w, x = x * rsqrt(
 * mean(x^2) + eps) * norm_w (per-head RMS-norm; the sum of squares follows the
 * reference's reduction order); then rotary embedding of the first `rot` channels
 * with cos/sin [S, rot/2] (fp32), MX_ROPE_INTERLEAVED pairing (2i, 2i+1) or
 * MX_ROPE_HALF pairing (i, i + rot/2); out[(s*H + h)*D + d] = bf16(x). Rules of
 * the reference's MX_CHECK: D even, D <= 256, rot even, rot <= D; S <= 0 is a no-op.
 * Results match the reference to bf16 rounding (its rsqrtf is an approximation). */
enum { MX_ROPE_NONE = 0, MX_ROPE_INTERLEAVED = 1, MX_ROPE_HALF = 2 };
int mx_head_norm_rope(const void* in, int64_t S, int64_t in_stride, int64_t col0, int H, int D, const float* norm_w,
                      float eps, const float* cos, const float* sin, int rot, int mode, void* out, void* stream);

/* Fused head_norm_rope + Sage attention. No single reference counterpart: it
 * replaces the sequence a DiT block runs before the quantized attention,
 * head_norm_rope(q), head_norm_rope(k) (src/kernels/ops.h:37-41, e.g.
 * src/models/minimax_h3/dit.cpp:210-211) then flash_attn_fp8 (attention.h:32-33),
 * without writing the normalised Q and K: q and k are the raw projections (rows
 * addressed by p's q_stride / kv_stride), each row gets the per-head RMS-norm
 * (q_norm / k_norm, NULL = none) and RoPE of the first `rot` channels with
 * cos/sin [row][rot/2] (Q row i uses table row i, K row j row j) and the bf16
 * rounding of head_norm_rope, then the Sage prologue. The workspace is
 * bit-identical to mx_head_norm_rope on q and k followed by mx_sage_quantize.
 * Needs the quantized path (mx_flash_attn_fp8_ok; D = 128) and, for
 * MX_ROPE_HALF, rot % 16 == 0: otherwise MX_E_UNSUPPORTED (there is no
 * fallback: the normalised tensors do not exist). */
typedef struct mx_qk_norm_rope {
  const float* q_norm;
  const float* k_norm;
  float eps;
  const float* cos;
  const float* sin;
  int rot, mode;
} mx_qk_norm_rope;
int mx_sage_quantize_norm_rope(const void* q, const void* k, const void* v, const mx_attn_params* p,
                               const mx_qk_norm_rope* nr, void* ws, void* stream);
int mx_flash_attn_fp8_norm_rope(const void* q, const void* k, const void* v, void* o, const mx_attn_params* p,
                                const mx_qk_norm_rope* nr, void* ws, void* stream);

/* ---- block-scaled GEMM (the DiT linears' low-precision path) ----
 * Reference: src/kernels/blockscale.h:12-37 (QMode, QMat, qmode_supported,
 * qdata_bytes, qscale_bytes, quantize_blockscaled, gemm_blockscaled; cuBLASLt in
 * blockscale.cu:134-216). MX_QMODE_MXFP8: e4m3 data, one UE8M0 (power-of-two)
 * scale per 32 K values, on gfx950's scaled MFMA. MX_QMODE_NVFP4: e2m1 data (two
 * per byte, low nibble first), one e4m3 scale per 16 K values and a per-tensor amax
 * (device float, written by quantize_blockscaled); gfx950's scaled MFMA has no
 * e4m3-per-16 form, so the GEMM dequantizes exactly to f16 in registers and runs
 * the f16 MFMA with fp32 accumulation and alpha = (amaxW / 2688) (amaxX / 2688).
 * Scale layout: the reference's 128x4 interleave (blockscale.cu:82, decoded by
 * tests/blockscale_test.cpp:15-17): scale (r, kb) at byte (r/128)*kbp*128 +
 * (kb/4)*512 + (r%32)*16 + ((r%128)/32)*4 + kb%4, kbp = K/vec rounded up to 4
 * (vec 32 MXFP8, 16 NVFP4), rows padded to 128; padding bytes hold 127 (1.0) for
 * MXFP8 and 0 for NVFP4. */
enum { MX_QMODE_BF16 = 0, MX_QMODE_MXFP8 = 1, MX_QMODE_NVFP4 = 2 };
int mx_qmode_supported(int mode, int device, int* supported);
size_t mx_qdata_bytes(int mode, int64_t rows, int64_t K);
size_t mx_qscale_bytes(int mode, int64_t rows, int64_t K);
/* Reference quantize_blockscaled (blockscale.cu:113-131): x [rows, K] bf16 with row
 * stride ldx -> q (MXFP8: [rows, K] e4m3, 16-byte aligned; NVFP4: [rows, K/2] e2m1
 * pairs, 8-byte aligned) and sf. K % 32 == 0, ldx % 8 == 0, x 16-byte aligned
 * (reference MX_CHECK). amax: NVFP4's per-tensor max |x| (device float, required);
 * unused for MXFP8 (may be NULL). */
int mx_quantize_blockscaled(int mode, const void* x, int64_t ldx, int64_t rows, int64_t K, void* q, void* sf,
                            float* amax, void* stream);
/* Reference gemm_blockscaled (blockscale.cu:134-216): Y[M, N] (bf16, row stride ldy)
 * = X[M, K] W[N, K]^T (+ Y when beta == 1), both quantized with the same mode; beta
 * must be 0 or 1. The QMat arguments are passed field by field (data, scales, amax);
 * wamax / xamax are the NVFP4 per-tensor amax values (required for NVFP4, ignored
 * for MXFP8). The reference's Ctx argument (cuBLASLt handle and workspace) becomes
 * the stream: these kernels need neither. */
int mx_gemm_blockscaled(int mode, const void* wq, const void* wsf, const float* wamax, const void* xq, const void* xsf,
                        const float* xamax, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, float beta,
                        void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MIROXEN_ATTN_H */

/*
 * CPU oracle for the DiT joint-attention hot path. TEST INFRASTRUCTURE ONLY:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker (or the timed CPU baseline). The
 * product path (miroxen_amd/) never links or calls it.
 *
 * Every routine restates the reference algorithm in plain C; the reference
 * file:line each one follows is cited beside it (paths are relative to the
 * reference repository root). Build: oracle/Makefile (gcc, -ffp-contract=off so
 * float expressions round exactly as written; no -ffast-math).
 *
 * Pinning (what fixes each routine independently of its own formula):
 *  - or_attention_f64: closed form softmax(s*QK^T)V in double; pinned in
 *    tests/test_oracle.py by a brute-force numpy float64 attention on tiny
 *    shapes, one-hot/uniform special cases and the mask-compaction invariant.
 *  - or_quant_rows / or_kv_stats: pinned by hand-worked vectors (amax=0,
 *    +/-amax -> +/-127, half-way rounding to even, padded rows -> 0) and an
 *    independent numpy restatement on random data.
 *  - or_e4m3: pinned by the OCP FP8 table (all 256 codes decode/encode round
 *    trip, half-way cases, saturation to 448, subnormals).
 *  - or_head_norm_rope: pinned by numpy closed forms (RMS-norm in float64, RoPE
 *    as complex multiplication), invariants (rotation preserves pair norms,
 *    rot = 0 and no norm is the identity, half mode = interleaved mode on
 *    permuted channels) and the butterfly order checked against a direct
 *    restatement of the reference's shuffle pattern.
 *  - or_f32_to_f16 / or_f16_to_f32: pinned against numpy's IEEE float16 cast
 *    (ties to even, subnormals, overflow) on hand cases and random values.
 *  - or_sage_emulate: pinned by closed forms on hand-built quantized operands
 *    (exact integer scores, power-of-two scales): two live keys whose second weight
 *    448 * 2^-H * 2^-g is not an e4m3 value (P rounded in acc, l over the unrounded
 *    weight, the 448 scale), a cross-tile rescale (alpha on l and acc) under the
 *    reference rule and the lazy rule, one live key, uniform scores; and by the
 *    reference gate (rel-RMS < 4 % vs exact attention, tests/attention_fp8_test.cpp:65).
 *  - or_mxfp8_quantize: pinned by the scale rule checked against float64
 *    ceil(log2(bmax / 448)) (independent of the frexp formulation), hand cases
 *    (zero block, bmax / 448 a power of two, just above one), exact round trips
 *    of e4m3 values times 2^k and the half-ulp error bound. Its scales come out
 *    in logical [rows][K/32] order; the reference's 128 x 4 interleave is
 *    oracle.mx_sf_offset (Python), pinned by hand-picked offsets of the
 *    reference decoder's formula and the bijection onto the padded buffer.
 *  - or_gemm_mxfp8: pinned by a numpy float64 dequantize-and-matmul and the
 *    identity-weight case (W = I with unit scales returns deq(X)).
 *  - or_e2m1: pinned by a nearest-value search over the e2m1 grid with ties to the
 *    even code (all midpoints), saturation and signs.
 *  - or_nvfp4_quantize: pinned by numpy's max |x| for amax, hand cases (the tensor's
 *    largest element gets scale 448 and code 6, a zero block scale 0 and codes 0,
 *    amax = 0 gives g = 1), the scale against e4m3 of float64 bmax / (6 g) and the
 *    element error bound (half an e2m1 step of the block, or saturation at 6).
 *  - or_gemm_nvfp4: pinned by a numpy float64 decode (the reference test's decoder,
 *    tests/blockscale_test.cpp:37-43) and matmul times alpha.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------- scalar helpers ---------- */

float or_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* float -> bf16, round to nearest even (NaN kept quiet). */
uint16_t or_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* OCP FP8 E4M3FN encoder (OCP 8-bit Floating Point Specification v1.0):
 * bias 7, no infinities, S.1111.111 = NaN, max finite 448. Round to nearest
 * even, saturate finite overflow to +/-448 (the reference's __NV_SATFINITE
 * conversion at src/kernels/attention_fp8.cu:119 and :187-188). */
uint8_t or_e4m3(float x) {
  if (isnan(x)) return 0x7f;
  uint8_t s = signbit(x) ? 0x80 : 0;
  double a = fabs((double)x);
  if (a >= 448.0) return s | 0x7e;
  /* quantum: 2^-9 in the subnormal range (a < 2^-6), else 2^(e-3) */
  int e;
  double q;
  if (a < 0.015625) {
    q = 1.0 / 512.0;
  } else {
    frexp(a, &e); /* a = m * 2^e, m in [0.5,1) -> floor(log2 a) = e-1 */
    q = ldexp(1.0, e - 1 - 3);
  }
  double n = a / q;           /* exact: q is a power of two */
  double r = floor(n);
  double frac = n - r;
  if (frac > 0.5 || (frac == 0.5 && fmod(r, 2.0) != 0.0)) r += 1.0;
  double v = r * q;
  if (v >= 448.0) return s | 0x7e;
  if (v == 0.0) return s;
  if (v < 0.015625) return s | (uint8_t)(v * 512.0);
  frexp(v, &e);
  int ex = e - 1;                                /* v in [2^ex, 2^(ex+1)) */
  int m = (int)(v / ldexp(1.0, ex) * 8.0) - 8;   /* 3 mantissa bits */
  return s | (uint8_t)(((ex + 7) << 3) | m);
}

float or_e4m3_to_f32(uint8_t c) {
  int s = c & 0x80, e = (c >> 3) & 15, m = c & 7;
  float v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf(1.0f + m / 8.0f, e - 7);
  return s ? -v : v;
}

/* IEEE binary16 of a float, round to nearest even (overflow -> inf, subnormals kept);
 * the build's split partials are stored in this format. Pinned in tests/test_oracle.py
 * against numpy's float16 conversion and hand cases. */
uint16_t or_f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const int e = (int)((u >> 23) & 0xff);
  uint32_t mant = u & 0x7fffffu;
  if (e == 0xff) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
  const int exp = e - 127 + 15;
  if (exp >= 31) return (uint16_t)(sign | 0x7c00u);
  if (exp <= 0) {
    if (exp < -10) return sign;
    mant |= 0x800000u;
    const int shift = 14 - exp;
    uint32_t half = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u), halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (half & 1u))) ++half;
    return (uint16_t)(sign | half);
  }
  uint32_t half = ((uint32_t)exp << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) ++half;  /* a carry may reach inf */
  return (uint16_t)(sign | half);
}

float or_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const int e = (h >> 10) & 0x1f;
  const uint32_t m = h & 0x3ffu;
  float f;
  if (e == 0) {
    f = (float)m * 5.9604644775390625e-8f; /* 2^-24 */
    return sign ? -f : f;
  }
  uint32_t u = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((uint32_t)(e - 15 + 127) << 23) | (m << 13));
  memcpy(&f, &u, 4);
  return f;
}

/* ---------- exact attention (double) ----------
 * Restates tests/attention_test.cu:64-98 (cpu_oracle): double dot products,
 * scale, subtract the row max, exp, normalise by the sum; 0 when the sum is 0.
 * Extended with the key-padding mask (kv_valid[key]==0 -> weight 0), causal
 * (key <= q_offset + row, tests/attention_test.cu:75) and GQA.
 * rows: the query rows to evaluate (n_rows of them); out: [n_rows][Hq][D] f32. */
void or_attention_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                      int Sq, int Skv, int Hq, int Hkv, int D, float scale,
                      int causal, int q_offset, int64_t q_stride, int64_t kv_stride,
                      const uint8_t* kv_valid, const int* rows, int n_rows, float* out,
                      int threads) {
  (void)Sq;
  double sc = scale == 0.f ? 1.0 / sqrt((double)D) : (double)scale;
  int group = Hq / Hkv;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
  for (int64_t job = 0; job < (int64_t)n_rows * Hq; ++job) {
    int ri = (int)(job / Hq), head = (int)(job % Hq);
    int row = rows[ri], kvh = head / group;
    int64_t end = Skv;
    if (causal) {
      int64_t last = (int64_t)q_offset + row + 1;
      end = last < 0 ? 0 : (last < Skv ? last : Skv);
    }
    double* w = (double*)malloc(sizeof(double) * (end > 0 ? end : 1));
    double* acc = (double*)calloc(D, sizeof(double));
    double mx = -INFINITY, sum = 0.0;
    const uint16_t* qr = q + (int64_t)row * q_stride + (int64_t)head * D;
    for (int64_t key = 0; key < end; ++key) {
      if (kv_valid && !kv_valid[key]) { w[key] = -INFINITY; continue; }
      const uint16_t* kr = k + key * kv_stride + (int64_t)kvh * D;
      double dot = 0.0;
      for (int d = 0; d < D; ++d) dot += (double)or_bf16_to_f32(qr[d]) * or_bf16_to_f32(kr[d]);
      w[key] = dot * sc;
      if (w[key] > mx) mx = w[key];
    }
    for (int64_t key = 0; key < end; ++key) {
      double e = w[key] == -INFINITY ? 0.0 : exp(w[key] - mx);
      w[key] = e;
      sum += e;
    }
    for (int64_t key = 0; key < end; ++key) {
      if (w[key] == 0.0) continue;
      const uint16_t* vr = v + key * kv_stride + (int64_t)kvh * D;
      for (int d = 0; d < D; ++d) acc[d] += w[key] * or_bf16_to_f32(vr[d]);
    }
    float* o = out + ((int64_t)ri * Hq + head) * D;
    for (int d = 0; d < D; ++d) o[d] = sum > 0.0 ? (float)(acc[d] / sum) : 0.f;
    free(w);
    free(acc);
  }
}

/* ---------- Sage prologue ---------- */

/* K per-channel mean and V per-channel abs-max.
 * Restates src/kernels/attention_fp8.cu:51-62 (kv_stats_kernel) with the
 * summation order fixed: s_b is a sequential float sum over block b's <= 256
 * tokens (:56-58), and kmean = sum over b ascending of (s_b / float(Skv))
 * starting from 0.f (:60, one legal atomicAdd order; the exact order when
 * Skv <= 256). vamax = max |v| (order independent, :61). */
void or_kv_stats(const uint16_t* k, const uint16_t* v, int Skv, int Hkv, int D,
                 int64_t kv_stride, float* kmean, float* vamax) {
  for (int h = 0; h < Hkv; ++h)
    for (int d = 0; d < D; ++d) {
      float mean = 0.f, am = 0.f;
      for (int64_t t0 = 0; t0 < Skv; t0 += 256) {
        int64_t t1 = t0 + 256 < Skv ? t0 + 256 : Skv;
        float s = 0.f;
        for (int64_t t = t0; t < t1; ++t) {
          s += or_bf16_to_f32(k[t * kv_stride + (int64_t)h * D + d]);
          float a = fabsf(or_bf16_to_f32(v[t * kv_stride + (int64_t)h * D + d]));
          am = a > am ? a : am;
        }
        mean += s / (float)Skv;
      }
      kmean[h * D + d] = mean;
      vamax[h * D + d] = am;
    }
}

/* Per-(head, G-row block) symmetric INT8 quantization.
 * Restates src/kernels/attention_fp8.cu:65-100 (quant_rows_kernel):
 * x' = bf16(x) - mean[c] (mean may be NULL), amax = max|x'| over the block,
 * inv = amax > 0 ? 127.f/amax : 0, q = rint(x'*inv) (round half even,
 * __float2int_rn at :96), scale = amax/127.f*mult (:99). Rows >= S are 0.
 * out: [H][s_pad][D] int8, scale_out: [H][s_pad/G] f32. */
void or_quant_rows(const uint16_t* x, int64_t stride, int S, int64_t s_pad, int H, int D, int G,
                   const float* mean, float mult, int8_t* out, float* scale_out) {
  float* buf = (float*)malloc(sizeof(float) * G * D);
  for (int h = 0; h < H; ++h)
    for (int64_t g = 0; g < s_pad / G; ++g) {
      float am = 0.f;
      for (int r = 0; r < G; ++r) {
        int64_t row = g * G + r;
        for (int c = 0; c < D; ++c) {
          float f = 0.f;
          if (row < S) {
            f = or_bf16_to_f32(x[row * stride + (int64_t)h * D + c]);
            if (mean) f = f - mean[h * D + c];
          }
          buf[r * D + c] = f;
          float a = fabsf(f);
          am = a > am ? a : am;
        }
      }
      float inv = am > 0.f ? 127.f / am : 0.f;
      for (int r = 0; r < G; ++r)
        for (int c = 0; c < D; ++c) {
          float p = buf[r * D + c] * inv;
          out[((int64_t)h * s_pad + g * G + r) * D + c] = (int8_t)(int)nearbyintf(p);
        }
      scale_out[(int64_t)h * (s_pad / G) + g] = am / 127.f * mult;
    }
  free(buf);
}

/* V -> e4m3 with per-channel scale 448/amax, transposed to [H][D][skv_pad].
 * Restates src/kernels/attention_fp8.cu:110-127 (v_quant_kernel): f = v*(448.f/a)
 * when the key exists and a > 0, else 0; SATFINITE e4m3. Keys are stored in
 * natural order (the reference's intra-32 key_pos permutation at :104-107 is an
 * operand-layout detail of its MMA, not part of the values). */
void or_v_quant(const uint16_t* v, int Skv, int Hkv, int D, int64_t kv_stride, int64_t skv_pad,
                const float* vamax, uint8_t* vt) {
  for (int h = 0; h < Hkv; ++h)
    for (int d = 0; d < D; ++d) {
      float a = vamax[h * D + d];
      for (int64_t key = 0; key < skv_pad; ++key) {
        float f = 0.f;
        if (key < Skv && a > 0.f) f = or_bf16_to_f32(v[key * kv_stride + (int64_t)h * D + d]) * (448.f / a);
        vt[((int64_t)h * D + d) * skv_pad + key] = or_e4m3(f);
      }
    }
}

/* ---------- Sage attention emulator ----------
 * Scalar restatement of the arithmetic of src/kernels/attention_fp8.cu:286-416
 * (fp8_attn_kernel, FP8 P.V path) over 64-key tiles:
 *   s = sum_d qi*ki (int32, exact)                                  :286-304
 *   sc = qs[row/16] * ks[tile]                                      :308
 *   im = max over the tile's live keys (integers), next = max(m, im*sc)  :322-327
 *     (or the lazy rule with headroom H, see below; H = 0 is the reference)
 *   alpha = 2^(m - next) (0 on the first tile)                      :328
 *   f = 2^(fma(bits(s + 0x4B400000), sc, nm)), nm = (log2 448 - H - next)
 *       - 12582912*sc; dead keys -> 0                                  :331-338
 *   l = l*alpha + sum f (unquantized f)                             :345
 *   acc = acc*alpha + sum e4m3(f) * e4m3(vt)  (fp32 accumulate)     :352, :374-402
 *   out = acc*vamax[d] * (1/(448*l)), 0 if l == 0                   :405-416
 * "Dead" keys are keys >= Skv (the reference's tail, :309-316) and keys with
 * kv_valid[key] == 0 (the build's key-padding mask). A tile with no live key for
 * a row leaves m, l and acc unchanged. The exponent follows the reference's
 * bit-trick formulation operation for operation (:331, :337).
 * exp2 here is libm's double exp2 rounded to float (the GPU uses v_exp_f32,
 * < 1 ulp). out: [n_rows][Hq][D] f32 (before the bf16 store). */
/* One key-tile range [t0, t1) of one (row, head): updates m, l, acc in place. */
static void or_sage_range(const int8_t* qr, float qscale, const int8_t* ki, const uint8_t* vt, const float* ksh,
                          int kvh, int Skv, int D, int64_t skv_pad, const uint8_t* kv_valid, const float* lut,
                          float headroom, int t0, int t1, float* m_io, float* l_io, float* acc) {
  const float L448 = 8.807354922057604f;
  float m = *m_io, l = *l_io;
  int32_t s[64];
  float f[64];
  for (int t = t0; t < t1; ++t) {
    const float sc = qscale * ksh[t];
    int live_any = 0;
    int32_t im = INT32_MIN;
    for (int j = 0; j < 64; ++j) {
      int64_t key = (int64_t)t * 64 + j;
      int live = key < Skv && (!kv_valid || kv_valid[key]);
      const int8_t* kr = ki + ((int64_t)kvh * skv_pad + key) * D;
      int32_t dot = 0;
      for (int d = 0; d < D; ++d) dot += (int32_t)qr[d] * (int32_t)kr[d];
      s[j] = live ? dot : INT32_MIN;
      if (live) { live_any = 1; if (dot > im) im = dot; }
    }
    if (!live_any) continue;
    const float tmax = (float)im * sc;
    /* headroom 0: next = max(m, tmax), the reference rule (:327). headroom H > 0:
     * lazy max, m moves only when the tile max exceeds it by more than H, and P
     * carries 2^-H so it stays <= 448 (this build's kernel uses H = 3). */
    float next = tmax > m + headroom ? tmax : m;
    float alpha = m == -INFINITY ? 0.f : (float)exp2((double)(m - next));
    m = next;
    /* exponent as the reference computes it (:331, :337): the int32 score is read as
     * the float 12582912 + s through its bits (s + 0x4B400000), one FMA with
     * nm = (log2 448 - H - next) - 12582912*sc (two float roundings). */
    const float nm = (L448 - headroom - next) - 12582912.f * sc;
    float ts = 0.f;
    for (int j = 0; j < 64; ++j) {
      if (s[j] == INT32_MIN) { f[j] = 0.f; continue; }
      int32_t biased = s[j] + 0x4B400000;
      float sb;
      memcpy(&sb, &biased, 4);
      f[j] = (float)exp2((double)fmaf(sb, sc, nm));
      ts += f[j];
    }
    l = l * alpha + ts;
    float p8[64];
    for (int j = 0; j < 64; ++j) p8[j] = lut[or_e4m3(f[j])];
    for (int d = 0; d < D; ++d) {
      const uint8_t* vr = vt + ((int64_t)kvh * D + d) * skv_pad + (int64_t)t * 64;
      float pv = 0.f;
      for (int j = 0; j < 64; ++j) pv += p8[j] * lut[vr[j]];
      acc[d] = acc[d] * alpha + pv;
    }
  }
  *m_io = m;
  *l_io = l;
}

/* split_full / split_parts / split_qt: the build's key-range split of the attention
 * grid (units = (head, split_qt-query tile), unit index head * ceil(Sq/split_qt) +
 * row/split_qt). Units
 * at or past split_full run as split_parts ranges of key tiles, [j*nt/P, (j+1)*nt/P),
 * each with its own m, l, acc; a part keeps o_j = fp16(acc_j / (448 l_j)); merged as
 * M = max m_j, w_j = 2^(m_j - M), c_j = l_j w_j, l = sum c_j, acc = sum (448 c_j) o_j
 * in part order. split_parts <= 1: no split. */
void or_sage_emulate(const int8_t* qi, const int8_t* ki, const uint8_t* vt, const float* qs,
                     const float* ks, const float* vamax, int Sq, int Skv, int Hq, int Hkv, int D,
                     int64_t sq_pad, int64_t skv_pad, const uint8_t* kv_valid, const int* rows,
                     int n_rows, float* out, int threads, float headroom, int split_full, int split_parts,
                     int split_qt) {
  const int group = Hq / Hkv;
  const int qt = split_qt > 0 ? split_qt : 256;
  const int ntq = (Sq + qt - 1) / qt;
  float lut[256];
  for (int c = 0; c < 256; ++c) lut[c] = or_e4m3_to_f32((uint8_t)c);
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
  for (int64_t job = 0; job < (int64_t)n_rows * Hq; ++job) {
    int ri = (int)(job / Hq), head = (int)(job % Hq), row = rows[ri], kvh = head / group;
    const int8_t* qr = qi + ((int64_t)head * sq_pad + row) * D;
    const float qscale = qs[(int64_t)head * (sq_pad / 16) + row / 16];
    const float* ksh = ks + (int64_t)kvh * (skv_pad / 64);
    const int ntiles = (int)((Skv + 63) / 64);
    const int unit = head * ntq + row / qt;
    const int parts = split_parts > 1 && unit >= split_full ? split_parts : 1;
    float* acc = (float*)calloc(D, sizeof(float));
    float* pa = (float*)calloc((size_t)parts * D, sizeof(float));
    float pm[8], pl[8];
    for (int j = 0; j < parts; ++j) {
      pm[j] = -INFINITY;
      pl[j] = 0.f;
      or_sage_range(qr, qscale, ki, vt, ksh, kvh, Skv, D, skv_pad, kv_valid, lut, headroom,
                    (int)((int64_t)j * ntiles / parts), (int)((int64_t)(j + 1) * ntiles / parts), &pm[j], &pl[j],
                    pa + (size_t)j * D);
    }
    float l = pl[0];
    if (parts == 1) {
      memcpy(acc, pa, sizeof(float) * D);
    } else {
      /* each part stores o_j = fp16(acc_j * (1 / (448 l_j))) (0 when l_j = 0) */
      for (int j = 0; j < parts; ++j) {
        const float inv = pl[j] > 0.f ? 1.f / (448.f * pl[j]) : 0.f;
        for (int d = 0; d < D; ++d) pa[(size_t)j * D + d] = or_f16_to_f32(or_f32_to_f16(pa[(size_t)j * D + d] * inv));
      }
      float mm = -INFINITY;
      for (int j = 0; j < parts; ++j) mm = fmaxf(mm, pm[j]);
      l = 0.f;
      for (int j = 0; j < parts; ++j) {
        const float w = mm == -INFINITY ? 0.f : (float)exp2((double)(pm[j] - mm));
        const float c = pl[j] * w;
        l += c;
        const float c448 = 448.f * c;
        for (int d = 0; d < D; ++d) acc[d] += c448 * pa[(size_t)j * D + d];
      }
    }
    float* o = out + ((int64_t)ri * Hq + head) * D;
    for (int d = 0; d < D; ++d) {
      float inv = l > 0.f ? 1.f / (448.f * l) : 0.f;
      o[d] = acc[d] * vamax[kvh * D + d] * inv;
    }
    free(pa);
    free(acc);
  }
}

/* ---------- head_norm_rope (reference src/kernels/ops.cu:87-119, :14-29) ----------
 * Per (token s, head h): x_d = bf16 in[s*in_stride + col0 + h*D + d]. If norm_w:
 * ss = the reference block_sum of x_d^2 over threads d < ceil(D/32)*32 (zeros
 * past D): inside each 32-thread warp an xor butterfly (offsets 16, 8, 4, 2, 1),
 * then the same butterfly over the warp partials padded to 32 slots;
 * x_d = x_d * rstd * norm_w[d] with rstd = 1/sqrt(ss/D + eps) (the reference
 * calls rsqrtf, an approximation; here the correctly rounded value). Then RoPE of
 * channels d < rot (mode 1: pairs (2i, 2i+1); mode 2: (i, i + rot/2)):
 * (a, b) -> (a c - b s, a s + b c) with c, s = cos/sin[s][pair]; output bf16. */
static float or_butterfly32(const float* x) { /* x[32] -> the xor-butterfly total */
  float a[32];
  memcpy(a, x, sizeof a);
  for (int o = 16; o > 0; o >>= 1) {
    float b[32];
    for (int l = 0; l < 32; ++l) b[l] = a[l] + a[l ^ o];
    memcpy(a, b, sizeof a);
  }
  return a[0];
}

void or_head_norm_rope(const uint16_t* in, int64_t S, int64_t in_stride, int64_t col0, int H, int D,
                       const float* norm_w, float eps, const float* cs, const float* sn, int rot, int mode,
                       uint16_t* out) {
  const int nwarp = (D + 31) / 32, half = rot / 2;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < S * H; ++r) {
    const int64_t s = r / H;
    const int h = (int)(r % H);
    float v[256], buf[256];
    for (int d = 0; d < nwarp * 32; ++d)
      v[d] = d < D ? or_bf16_to_f32(in[s * in_stride + col0 + (int64_t)h * D + d]) : 0.f;
    if (norm_w) {
      float part[32] = {0};
      for (int w = 0; w < nwarp; ++w) {
        float sq[32];
        for (int l = 0; l < 32; ++l) sq[l] = v[w * 32 + l] * v[w * 32 + l];
        part[w] = or_butterfly32(sq);
      }
      const float ss = or_butterfly32(part);
      const float rstd = (float)(1.0 / sqrt((double)(ss / (float)D + eps)));
      for (int d = 0; d < D; ++d) v[d] = v[d] * rstd * norm_w[d];
    }
    for (int d = 0; d < D; ++d) buf[d] = v[d];
    if (mode != 0 && rot > 0) {
      for (int d = 0; d < rot; ++d) {
        int pair, idx;
        float other;
        if (mode == 1) {
          pair = d >> 1;
          idx = d & 1;
          other = buf[d ^ 1];
        } else {
          pair = d < half ? d : d - half;
          idx = d < half ? 0 : 1;
          other = buf[d < half ? d + half : d - half];
        }
        const float c = cs[s * half + pair], si = sn[s * half + pair];
        v[d] = idx == 0 ? v[d] * c - other * si : other * si + v[d] * c;
      }
    }
    for (int d = 0; d < D; ++d) out[r * D + d] = or_f32_to_bf16(v[d]);
  }
}

int or_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ---------- MXFP8 block-scaled quantizer (reference src/kernels/blockscale.cu:69-108) ----------
 * Per row r and 32-value block kb of x (bf16, row stride ldx): bmax = max |v|;
 * e = -127 when bmax == 0, else frexpf(bmax / 448.f) = mant * 2^ex and e = ex - 1
 * when mant == 0.5 (bmax / 448 a power of two), ex otherwise, clamped to [-127, 127]
 * (:95-101): the smallest power of two with bmax / 2^e <= 448. q = e4m3 SATFINITE of
 * v * 2^-e (:102-103, the exact power of two the reference's exp2f(-e) returns),
 * scale byte e + 127. q [rows][K] dense; sf [rows][K/32] (this library's layout). */
void or_mxfp8_quantize(const uint16_t* x, int64_t ldx, int64_t rows, int64_t K, uint8_t* q, uint8_t* sf) {
  const int64_t nkb = K / 32;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t kb = 0; kb < nkb; ++kb) {
      float v[32], bmax = 0.f;
      for (int j = 0; j < 32; ++j) {
        v[j] = or_bf16_to_f32(x[r * ldx + kb * 32 + j]);
        if (fabsf(v[j]) > bmax) bmax = fabsf(v[j]);
      }
      int e = -127;
      if (bmax > 0.f) {
        int ex;
        const float t = bmax / 448.f;
        const float mant = frexpf(t, &ex);
        e = mant == 0.5f ? ex - 1 : ex;
        e = e < -127 ? -127 : (e > 127 ? 127 : e);
      }
      const float inv = ldexpf(1.f, -e);
      for (int j = 0; j < 32; ++j) q[r * K + kb * 32 + j] = or_e4m3(v[j] * inv);
      sf[r * nkb + kb] = (uint8_t)(e + 127);
    }
}

/* Y[m][n] = sum_k deq(X[m][k]) * deq(W[n][k]) in double, deq(c) = e4m3(c) * 2^(s - 127)
 * with s the block's scale byte (sf [rows][K/32]); out [M][N] as float. */
void or_gemm_mxfp8(const uint8_t* wq, const uint8_t* wsf, const uint8_t* xq, const uint8_t* xsf, int64_t M,
                   int64_t N, int64_t K, float* out, int threads) {
  const int64_t nkb = K / 32;
  float lut[256];
  for (int c = 0; c < 256; ++c) lut[c] = or_e4m3_to_f32((uint8_t)c);
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0;
      for (int64_t kb = 0; kb < nkb; ++kb) {
        double blk = 0.0;
        for (int j = 0; j < 32; ++j)
          blk += (double)lut[xq[m * K + kb * 32 + j]] * (double)lut[wq[n * K + kb * 32 + j]];
        acc += blk * ldexp(1.0, (int)xsf[m * nkb + kb] - 127) * ldexp(1.0, (int)wsf[n * nkb + kb] - 127);
      }
      out[m * N + n] = (float)acc;
    }
}

/* ---------- NVFP4 (reference src/kernels/blockscale.cu, NVFP4 branch) ----------
 * e2m1 (OCP FP4: 1 sign, 2 exponent, 1 mantissa bit; magnitudes 0, 0.5, 1, 1.5, 2, 3,
 * 4, 6) of x, rounded to the nearest magnitude with ties to the even code and
 * saturated to 6, as the reference's threshold sum (blockscale.cu:38-42): a
 * magnitude code counts the thresholds 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5 that |x|
 * passes, strictly above the ones whose lower neighbour has an even code (0.25,
 * 1.25, 2.5, 5) and at or above the others. Sign bit 8 for x < 0 (so -0 and NaN
 * encode with sign 0). */
uint8_t or_e2m1(float x) {
  const float a = fabsf(x);
  const uint8_t c = (uint8_t)((a > 0.25f) + (a >= 0.75f) + (a > 1.25f) + (a >= 1.75f) + (a > 2.5f) + (a >= 3.5f) +
                              (a > 5.f));
  return (uint8_t)(c | (x < 0.f ? 8 : 0));
}

float or_e2m1_to_f32(uint8_t c) {
  static const float mag[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
  const float v = mag[c & 7];
  return (c & 8) ? -v : v;
}

/* quantize_blockscaled(NVFP4) (blockscale.cu:113-131 with amax_kernel :45-67 and
 * quant_kernel's NVFP4 branch :69-93): amax = max |x| over the tensor; g = amax / (6 *
 * 448) (1 when amax = 0); per 16-value block se = e4m3(bmax / (6 g)) (saturating, round
 * to nearest even), sd = float(se) g, inv = 1 / sd (0 when sd = 0), code j = e2m1(x_j
 * inv); two codes per byte, the lower-index value in the low nibble. sf: logical
 * [rows][K/16] e4m3 bytes. Float arithmetic in the reference's order. */
void or_nvfp4_quantize(const uint16_t* x, int64_t ldx, int64_t rows, int64_t K, uint8_t* q, uint8_t* sf,
                       float* amax_out) {
  float amax = 0.f;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t k = 0; k < K; ++k) {
      const float a = fabsf(or_bf16_to_f32(x[r * ldx + k]));
      if (a > amax) amax = a;
    }
  *amax_out = amax;
  const float g = amax > 0.f ? amax / (6.f * 448.f) : 1.f;
  const float inv6g = 1.f / (6.f * g);
  const int64_t nkb = K / 16;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t kb = 0; kb < nkb; ++kb) {
      float v[16], bmax = 0.f;
      for (int j = 0; j < 16; ++j) {
        v[j] = or_bf16_to_f32(x[r * ldx + kb * 16 + j]);
        if (fabsf(v[j]) > bmax) bmax = fabsf(v[j]);
      }
      const uint8_t se = or_e4m3(bmax * inv6g);
      const float sd = or_e4m3_to_f32(se) * g;
      const float inv = sd > 0.f ? 1.f / sd : 0.f;
      uint8_t* dst = q + (r * K + kb * 16) / 2;
      for (int j = 0; j < 8; ++j)
        dst[j] = (uint8_t)(or_e2m1(v[2 * j] * inv) | (or_e2m1(v[2 * j + 1] * inv) << 4));
      sf[r * nkb + kb] = se;
    }
}

/* gemm_blockscaled(NVFP4) (blockscale.cu:134-216: cuBLASLt with VEC16_UE4M3 block
 * scales and alpha = gW gX from alpha_kernel :111-115): Y[m][n] = alpha * sum_k
 * (e2m1 x se)_X (e2m1 x se)_W, the sum in double, alpha in float as the reference
 * computes it. sf [rows][K/16] logical order. out [M][N] float. */
void or_gemm_nvfp4(const uint8_t* wq, const uint8_t* wsf, float wamax, const uint8_t* xq, const uint8_t* xsf,
                   float xamax, int64_t M, int64_t N, int64_t K, float* out, int threads) {
  const int64_t nkb = K / 16;
  const float gw = wamax > 0.f ? wamax / (6.f * 448.f) : 1.f, gx = xamax > 0.f ? xamax / (6.f * 448.f) : 1.f;
  const float alpha = gw * gx;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0;
      for (int64_t kb = 0; kb < nkb; ++kb) {
        double blk = 0.0;
        for (int j = 0; j < 16; ++j) {
          const int64_t k = kb * 16 + j;
          const uint8_t cx = (uint8_t)((xq[(m * K + k) / 2] >> ((k & 1) * 4)) & 15);
          const uint8_t cw = (uint8_t)((wq[(n * K + k) / 2] >> ((k & 1) * 4)) & 15);
          blk += (double)or_e2m1_to_f32(cx) * (double)or_e2m1_to_f32(cw);
        }
        acc += blk * (double)or_e4m3_to_f32(xsf[m * nkb + kb]) * (double)or_e4m3_to_f32(wsf[n * nkb + kb]);
      }
      out[m * N + n] = (float)(acc * (double)alpha);
    }
}


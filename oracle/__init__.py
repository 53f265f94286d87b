"""CPU oracle for the DiT joint-attention hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or the timed CPU
baseline).  The product path (``miroxen_amd``) never imports it.

Thin ctypes wrapper over ``oracle/oracle.c`` (built by ``oracle/Makefile`` into
``oracle/liboracle.so``).  Tensors are numpy arrays; bf16 tensors are passed as
their raw ``uint16`` bit patterns.  The reference file:line each routine follows
is cited in ``oracle.c``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE, "-B"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.or_f32_to_bf16.restype = ctypes.c_uint16
        L.or_f32_to_bf16.argtypes = [_f]
        L.or_bf16_to_f32.restype = _f
        L.or_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_e4m3.restype = ctypes.c_uint8
        L.or_e4m3.argtypes = [_f]
        L.or_e4m3_to_f32.restype = _f
        L.or_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_f16.argtypes = [_f]
        L.or_f16_to_f32.restype = _f
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_attention_f64.restype = None
        L.or_attention_f64.argtypes = [_p, _p, _p, _i, _i, _i, _i, _i, _f, _i, _i, _i64, _i64,
                                       _p, _p, _i, _p, _i]
        L.or_kv_stats.restype = None
        L.or_kv_stats.argtypes = [_p, _p, _i, _i, _i, _i64, _p, _p]
        L.or_quant_rows.restype = None
        L.or_quant_rows.argtypes = [_p, _i64, _i, _i64, _i, _i, _i, _p, _f, _p, _p]
        L.or_v_quant.restype = None
        L.or_v_quant.argtypes = [_p, _i, _i, _i, _i64, _i64, _p, _p]
        L.or_sage_emulate.restype = None
        L.or_sage_emulate.argtypes = [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i64, _i64,
                                      _p, _p, _i, _p, _i, _f, _i, _i, _i]
        L.or_head_norm_rope.restype = None
        L.or_head_norm_rope.argtypes = [_p, _i64, _i64, _i64, _i, _i, _p, _f, _p, _p, _i, _i, _p]
        L.or_mxfp8_quantize.restype = None
        L.or_mxfp8_quantize.argtypes = [_p, _i64, _i64, _i64, _p, _p]
        L.or_gemm_mxfp8.restype = None
        L.or_gemm_mxfp8.argtypes = [_p, _p, _p, _p, _i64, _i64, _i64, _p, _i]
        L.or_e2m1.restype = ctypes.c_uint8
        L.or_e2m1.argtypes = [_f]
        L.or_e2m1_to_f32.restype = _f
        L.or_e2m1_to_f32.argtypes = [ctypes.c_uint8]
        L.or_nvfp4_quantize.restype = None
        L.or_nvfp4_quantize.argtypes = [_p, _i64, _i64, _i64, _p, _p, _p]
        L.or_gemm_nvfp4.restype = None
        L.or_gemm_nvfp4.argtypes = [_p, _p, _f, _p, _p, _f, _i64, _i64, _i64, _p, _i]
        L.or_num_threads.restype = _i
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bits (vectorised restatement of or_f32_to_bf16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3(x: float) -> int:
    return int(lib().or_e4m3(float(x)))


def f16(x: float) -> int:
    """IEEE binary16 bits of x, round to nearest even (the split partials' format)."""
    return int(lib().or_f32_to_f16(float(x)))


def f16_to_f32(h: int) -> float:
    return float(lib().or_f16_to_f32(int(h)))


def e4m3_to_f32(c: int) -> float:
    return float(lib().or_e4m3_to_f32(int(c)))


def attention_f64(q, k, v, Sq, Skv, Hq, Hkv, D, scale=0.0, causal=0, q_offset=0,
                  q_stride=0, kv_stride=0, kv_valid=None, rows=None, threads=0):
    """Exact attention (double accumulation) on selected query rows -> [rows, Hq, D] f32."""
    q = _c(q, np.uint16); k = _c(k, np.uint16); v = _c(v, np.uint16)
    q_stride = q_stride or Hq * D
    kv_stride = kv_stride or Hkv * D
    rows = np.arange(Sq, dtype=np.int32) if rows is None else _c(rows, np.int32)
    mask = None if kv_valid is None else _c(kv_valid, np.uint8)
    out = np.zeros((len(rows), Hq, D), np.float32)
    lib().or_attention_f64(_ptr(q), _ptr(k), _ptr(v), Sq, Skv, Hq, Hkv, D, scale, causal,
                           q_offset, q_stride, kv_stride, _ptr(mask), _ptr(rows), len(rows),
                           _ptr(out), threads)
    return out


def kv_stats(k, v, Skv, Hkv, D, kv_stride=0):
    k = _c(k, np.uint16); v = _c(v, np.uint16)
    kv_stride = kv_stride or Hkv * D
    km = np.zeros((Hkv, D), np.float32); va = np.zeros((Hkv, D), np.float32)
    lib().or_kv_stats(_ptr(k), _ptr(v), Skv, Hkv, D, kv_stride, _ptr(km), _ptr(va))
    return km, va


def quant_rows(x, stride, S, s_pad, H, D, G, mean, mult):
    x = _c(x, np.uint16)
    mean = None if mean is None else _c(mean, np.float32)
    out = np.zeros((H, s_pad, D), np.int8)
    sc = np.zeros((H, s_pad // G), np.float32)
    lib().or_quant_rows(_ptr(x), stride, S, s_pad, H, D, G, _ptr(mean), float(mult), _ptr(out), _ptr(sc))
    return out, sc


def v_quant(v, Skv, Hkv, D, kv_stride, skv_pad, vamax):
    v = _c(v, np.uint16); vamax = _c(vamax, np.float32)
    vt = np.zeros((Hkv, D, skv_pad), np.uint8)
    lib().or_v_quant(_ptr(v), Skv, Hkv, D, kv_stride, skv_pad, _ptr(vamax), _ptr(vt))
    return vt


# Lazy-max headroom of the GPU Sage kernel (log2 units); 0 = reference exact-max rule.
KERNEL_HEADROOM = 3.0


def sage_emulate(qi, ki, vt, qs, ks, vamax, Sq, Skv, Hq, Hkv, D, kv_valid=None, rows=None, threads=0,
                 headroom=0.0, split=None):
    """split = (split_full, split_parts[, split_qt]): units (head, split_qt-query tile,
    256 by default) at or past split_full are evaluated as split_parts key ranges and
    merged (the kernel's grid balancing); None = sequential over all keys, as the
    reference."""
    full, parts, qt = (tuple(split) + (256,))[:3] if split else (0, 1, 256)
    if parts > 8:
        raise ValueError("at most 8 split parts")
    qi = _c(qi, np.int8); ki = _c(ki, np.int8); vt = _c(vt, np.uint8)
    qs = _c(qs, np.float32); ks = _c(ks, np.float32); vamax = _c(vamax, np.float32)
    sq_pad = qi.shape[1]; skv_pad = ki.shape[1]
    rows = np.arange(Sq, dtype=np.int32) if rows is None else _c(rows, np.int32)
    mask = None if kv_valid is None else _c(kv_valid, np.uint8)
    out = np.zeros((len(rows), Hq, D), np.float32)
    lib().or_sage_emulate(_ptr(qi), _ptr(ki), _ptr(vt), _ptr(qs), _ptr(ks), _ptr(vamax), Sq, Skv,
                          Hq, Hkv, D, sq_pad, skv_pad, _ptr(mask), _ptr(rows), len(rows),
                          _ptr(out), threads, float(headroom), int(full), int(parts), int(qt))
    return out


def sage_reference(q, k, v, Sq, Skv, Hq, Hkv, D, scale=0.0, q_stride=0, kv_stride=0,
                   kv_valid=None, rows=None, q_group=16, threads=0, headroom=0.0):
    """Full Sage pipeline on the CPU: prologue (kv_stats, Q/K int8, V e4m3) + emulator.

    Returns (out [rows,Hq,D] f32, dict of quantized tensors)."""
    q_stride = q_stride or Hq * D
    kv_stride = kv_stride or Hkv * D
    scale = scale or 1.0 / np.sqrt(np.float32(D))
    sq_pad = (Sq + 255) // 256 * 256
    skv_pad = (Skv + 63) // 64 * 64
    km, va = kv_stats(k, v, Skv, Hkv, D, kv_stride)
    mult = np.float32(np.float32(scale) * np.float32(1.4426950408889634))
    qi, qs = quant_rows(q, q_stride, Sq, sq_pad, Hq, D, q_group, None, mult)
    ki, ks = quant_rows(k, kv_stride, Skv, skv_pad, Hkv, D, 64, km, 1.0)
    vt = v_quant(v, Skv, Hkv, D, kv_stride, skv_pad, va)
    out = sage_emulate(qi, ki, vt, qs, ks, va, Sq, Skv, Hq, Hkv, D, kv_valid, rows, threads, headroom)
    return out, dict(qi=qi, qs=qs, ki=ki, ks=ks, vt=vt, km=km, va=va)


def e2m1(x: float) -> int:
    return int(lib().or_e2m1(float(x)))


def e2m1_to_f32(c: int) -> float:
    return float(lib().or_e2m1_to_f32(int(c)))


def nvfp4_quantize(x, rows, K, ldx=0):
    """NVFP4 quantizer (reference blockscale.cu:45-93, :113-131): x bf16 bits [rows, ldx]
    -> (q uint8 [rows, K/2] two e2m1 codes per byte, low nibble first; sf uint8
    [rows, K/16] e4m3, logical order; amax float)."""
    x = _c(x, np.uint16)
    ldx = ldx or K
    q = np.zeros((rows, K // 2), np.uint8)
    sf = np.zeros((rows, K // 16), np.uint8)
    amax = np.zeros(1, np.float32)
    lib().or_nvfp4_quantize(_ptr(x), ldx, rows, K, _ptr(q), _ptr(sf), _ptr(amax))
    return q, sf, float(amax[0])


def gemm_nvfp4(wq, wsf, wamax, xq, xsf, xamax, M, N, K, threads=0):
    """Y[M, N] = alpha deq(X) deq(W)^T (sum in float64, alpha = gW gX in float)."""
    wq = _c(wq, np.uint8); wsf = _c(wsf, np.uint8); xq = _c(xq, np.uint8); xsf = _c(xsf, np.uint8)
    out = np.zeros((M, N), np.float32)
    lib().or_gemm_nvfp4(_ptr(wq), _ptr(wsf), float(wamax), _ptr(xq), _ptr(xsf), float(xamax), M, N, K, _ptr(out),
                        threads)
    return out


def num_threads() -> int:
    return int(lib().or_num_threads())


def head_norm_rope(inp, S, in_stride, col0, H, D, norm_w=None, eps=0.0, cos=None, sin=None, rot=0, mode=0):
    """Reference head_norm_rope (ops.cu:87-119) -> bf16 bits [S, H, D]."""
    inp = _c(inp, np.uint16)
    nw = None if norm_w is None else _c(norm_w, np.float32)
    cs = None if cos is None else _c(cos, np.float32)
    sn = None if sin is None else _c(sin, np.float32)
    out = np.zeros((S, H, D), np.uint16)
    lib().or_head_norm_rope(_ptr(inp), S, in_stride, col0, H, D, _ptr(nw), float(eps), _ptr(cs), _ptr(sn),
                            rot, mode, _ptr(out))
    return out


def mxfp8_quantize(x, rows, K, ldx=0):
    """MXFP8 quantizer (reference blockscale.cu:69-108): x bf16 bits [rows, ldx] ->
    (q uint8 [rows, K] e4m3, sf uint8 [rows, K/32] UE8M0, logical order; the device
    buffer's interleaved order is mx_scale_pack / mx_scale_unpack)."""
    x = _c(x, np.uint16)
    ldx = ldx or K
    q = np.zeros((rows, K), np.uint8)
    sf = np.zeros((rows, K // 32), np.uint8)
    lib().or_mxfp8_quantize(_ptr(x), ldx, rows, K, _ptr(q), _ptr(sf))
    return q, sf


def mx_sf_offset(r, kb, nkb_pad):
    """Byte offset of scale (row r, K block kb) in the block-scaled scale buffer: the
    128 x 4 interleaved tiles of the reference (quantizer src/kernels/blockscale.cu:82,
    decoder tests/blockscale_test.cpp:15-17). Each 128-row band holds nkb_pad / 4 tiles of
    512 bytes; inside a tile, row r % 32 owns 16 bytes, split into four 4-byte groups by
    (r % 128) / 32, and kb % 4 picks the byte."""
    r = np.asarray(r, np.int64); kb = np.asarray(kb, np.int64)
    return (r // 128) * nkb_pad * 128 + (kb // 4) * 512 + (r % 32) * 16 + (r % 128) // 32 * 4 + kb % 4


def mx_scale_pack(sf, rows, K, fill=127, vec=32):
    """Logical scales [rows, K/vec] -> the interleaved buffer (pad128(rows) x pad4(K/vec)
    bytes; vec 32 for MXFP8, 16 for NVFP4); padding positions hold `fill`."""
    nkb = K // vec
    nkp = (nkb + 3) // 4 * 4
    buf = np.full(((rows + 127) // 128 * 128) * nkp, fill, np.uint8)
    r, kb = np.meshgrid(np.arange(rows), np.arange(nkb), indexing="ij")
    buf[mx_sf_offset(r, kb, nkp)] = sf
    return buf


def mx_scale_unpack(buf, rows, K, vec=32):
    """The interleaved scale buffer -> logical scales [rows, K/vec]."""
    nkb = K // vec
    nkp = (nkb + 3) // 4 * 4
    r, kb = np.meshgrid(np.arange(rows), np.arange(nkb), indexing="ij")
    return np.asarray(buf, np.uint8).reshape(-1)[mx_sf_offset(r, kb, nkp)]


def gemm_mxfp8(wq, wsf, xq, xsf, M, N, K, threads=0):
    """Y[M, N] = deq(X) deq(W)^T in float64 (returned as float32)."""
    wq = _c(wq, np.uint8); wsf = _c(wsf, np.uint8); xq = _c(xq, np.uint8); xsf = _c(xsf, np.uint8)
    out = np.zeros((M, N), np.float32)
    lib().or_gemm_mxfp8(_ptr(wq), _ptr(wsf), _ptr(xq), _ptr(xsf), M, N, K, _ptr(out), threads)
    return out


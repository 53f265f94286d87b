"""ctypes binding of libmiroxen_attn.so (the C ABI in include/miroxen_attn.h).

The library is built in-tree by miroxen_amd/build.py; loading fails loudly when it
is missing — there is no CPU or PyTorch fallback for the product path.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libmiroxen_attn.so")

MX_OK, MX_E_INVALID, MX_E_HIP, MX_E_UNSUPPORTED = 0, -1, -2, -3

# Exported symbols, in header order (tests check every one is exported).
SYMBOLS = (
    "mx_flash_attn", "mx_flash_attn_fp8_workspace", "mx_flash_attn_fp8_supported",
    "mx_flash_attn_fp8_ok", "mx_flash_attn_fp8", "mx_flash_attn_uses_mfma", "mx_flash_attn_split_plan",
    "mx_flash_attn_fp8_noalloc",
    "mx_attn_reference", "mx_sage_layout_of",
    "mx_sage_quantize", "mx_sage_attend", "mx_last_error", "mx_version", "mx_head_norm_rope",
    "mx_sage_quantize_norm_rope", "mx_flash_attn_fp8_norm_rope", "mx_sage_quantize_qgroup", "mx_sage_prologue_wait_ticks",
    "mx_qmode_supported", "mx_qdata_bytes", "mx_qscale_bytes", "mx_quantize_blockscaled", "mx_gemm_blockscaled",
)


class CParams(ctypes.Structure):
    """mx_attn_params (reference AttnParams, src/kernels/attention.h:12-18, + kv_valid)."""
    _fields_ = [
        ("Sq", ctypes.c_int), ("Skv", ctypes.c_int), ("Hq", ctypes.c_int), ("Hkv", ctypes.c_int),
        ("D", ctypes.c_int), ("scale", ctypes.c_float), ("causal", ctypes.c_int),
        ("q_offset", ctypes.c_int), ("q_stride", ctypes.c_int64), ("kv_stride", ctypes.c_int64),
        ("o_stride", ctypes.c_int64), ("kv_valid", ctypes.c_void_p),
    ]


class CNormRope(ctypes.Structure):
    """mx_qk_norm_rope: per-head RMS-norm weights of Q and K, eps, RoPE tables and mode."""
    _fields_ = [("q_norm", ctypes.c_void_p), ("k_norm", ctypes.c_void_p), ("eps", ctypes.c_float),
                ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p), ("rot", ctypes.c_int), ("mode", ctypes.c_int)]


class CLayout(ctypes.Structure):
    _fields_ = [("sq_pad", ctypes.c_int64), ("skv_pad", ctypes.c_int64)] + [
        (n, ctypes.c_size_t) for n in ("qi", "ki", "vt", "qs", "ks", "km", "va", "part", "split", "cnt", "total")] + [
        ("split_units", ctypes.c_int), ("split_parts", ctypes.c_int), ("split_qt", ctypes.c_int),
        ("tab", ctypes.c_size_t), ("flg", ctypes.c_size_t)]


_lib = None


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"miroxen_amd: {LIB_PATH} is not built; run `python -m miroxen_amd.build`")
    L = ctypes.CDLL(LIB_PATH)
    vp, P = ctypes.c_void_p, ctypes.POINTER(CParams)
    ip = ctypes.POINTER(ctypes.c_int)
    sig = {
        "mx_flash_attn": ([vp, vp, vp, vp, P, vp], ctypes.c_int),
        "mx_flash_attn_fp8_workspace": ([P], ctypes.c_size_t),
        "mx_flash_attn_fp8_supported": ([ctypes.c_int, ip], ctypes.c_int),
        "mx_flash_attn_fp8_ok": ([vp, vp, vp, vp, P, ip], ctypes.c_int),
        "mx_flash_attn_fp8": ([vp, vp, vp, vp, P, vp, vp], ctypes.c_int),
        "mx_flash_attn_fp8_noalloc": ([vp, vp, vp, vp, P, vp], ctypes.c_int),
        "mx_flash_attn_uses_mfma": ([vp, vp, vp, vp, P, ip], ctypes.c_int),
        "mx_flash_attn_split_plan": ([P, ctypes.c_int, ip, ip, ip], ctypes.c_int),
        "mx_attn_reference": ([vp, vp, vp, vp, P, vp], ctypes.c_int),
        "mx_sage_layout_of": ([P, ctypes.POINTER(CLayout)], ctypes.c_int),
        "mx_sage_quantize": ([vp, vp, vp, P, vp, vp], ctypes.c_int),
        "mx_sage_quantize_qgroup": ([vp, vp, vp, P, vp, ctypes.c_int, vp], ctypes.c_int),
        "mx_sage_prologue_wait_ticks": ([ctypes.c_int64], ctypes.c_int),
        "mx_sage_attend": ([vp, P, vp, vp], ctypes.c_int),
        "mx_last_error": ([], ctypes.c_char_p),
        "mx_version": ([], ctypes.c_char_p),
        "mx_head_norm_rope": ([vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int, vp,
                               ctypes.c_float, vp, vp, ctypes.c_int, ctypes.c_int, vp, vp], ctypes.c_int),
        "mx_sage_quantize_norm_rope": ([vp, vp, vp, P, ctypes.POINTER(CNormRope), vp, vp], ctypes.c_int),
        "mx_flash_attn_fp8_norm_rope": ([vp, vp, vp, vp, P, ctypes.POINTER(CNormRope), vp, vp], ctypes.c_int),
        "mx_qmode_supported": ([ctypes.c_int, ctypes.c_int, ip], ctypes.c_int),
        "mx_qdata_bytes": ([ctypes.c_int, ctypes.c_int64, ctypes.c_int64], ctypes.c_size_t),
        "mx_qscale_bytes": ([ctypes.c_int, ctypes.c_int64, ctypes.c_int64], ctypes.c_size_t),
        "mx_quantize_blockscaled": ([ctypes.c_int, vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, vp, vp, vp,
                                     vp], ctypes.c_int),
        "mx_gemm_blockscaled": ([ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, ctypes.c_int64, ctypes.c_int64,
                                 ctypes.c_int64, ctypes.c_int64, ctypes.c_float, vp], ctypes.c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes, fn.restype = args, res
    _lib = L
    return L


def check(rc: int) -> None:
    """Raise like the reference's MX_CHECK / MX_CUDA (std::runtime_error)."""
    if rc != MX_OK:
        msg = load().mx_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"miroxen_amd error {rc}")

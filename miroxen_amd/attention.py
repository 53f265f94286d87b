"""Host-side mirror of the reference attention API (src/kernels/attention.h:12-39).

Same names, argument meaning and error behaviour as the reference's free
functions; tensors are torch tensors on the current HIP device (or raw device
addresses as ints). Invalid arguments raise RuntimeError, the Python face of the
reference's std::runtime_error. Everything runs in libmiroxen_attn.so.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

from . import _lib


@dataclass
class AttnParams:
    """Reference AttnParams (src/kernels/attention.h:12-18) + key-padding mask.

    scale == 0 -> 1/sqrt(D); strides of 0 -> dense H*D; kv_valid: uint8 [Skv] device
    tensor (0 = padded key) or None."""
    Sq: int = 0
    Skv: int = 0
    Hq: int = 0
    Hkv: int = 0
    D: int = 0
    scale: float = 0.0
    causal: int = 0
    q_offset: int = 0
    q_stride: int = 0
    kv_stride: int = 0
    o_stride: int = 0
    kv_valid: object = None

    def c(self) -> _lib.CParams:
        return _lib.CParams(self.Sq, self.Skv, self.Hq, self.Hkv, self.D, self.scale, self.causal,
                            self.q_offset, self.q_stride, self.kv_stride, self.o_stride,
                            _addr(self.kv_valid))


def _addr(t) -> Optional[int]:
    if t is None:
        return None
    if isinstance(t, int):
        return t or None
    return t.data_ptr() or None


def _stream(stream) -> Optional[int]:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream or None
    if isinstance(stream, int):
        return stream or None
    return stream.cuda_stream or None


def flash_attn(q, k, v, o, p: AttnParams, stream=None) -> None:
    """Reference mx::flash_attn (src/kernels/attention.cu:409-417)."""
    c = p.c()
    _lib.check(_lib.load().mx_flash_attn(_addr(q), _addr(k), _addr(v), _addr(o), ctypes.byref(c),
                                         _stream(stream)))


def attn_reference(q, k, v, o, p: AttnParams, stream=None) -> None:
    """Reference mx::attn_reference (src/kernels/attention.cu:419-423): naive fp32 GPU attention."""
    c = p.c()
    _lib.check(_lib.load().mx_attn_reference(_addr(q), _addr(k), _addr(v), _addr(o), ctypes.byref(c),
                                             _stream(stream)))


def flash_attn_fp8_workspace(p: AttnParams) -> int:
    """Reference mx::flash_attn_fp8_workspace (src/kernels/attention_fp8.cu:471-473)."""
    c = p.c()
    return int(_lib.load().mx_flash_attn_fp8_workspace(ctypes.byref(c)))


def flash_attn_fp8_supported(device: int) -> bool:
    """Reference mx::flash_attn_fp8_supported (src/kernels/attention_fp8.cu:475-482)."""
    out = ctypes.c_int(0)
    _lib.check(_lib.load().mx_flash_attn_fp8_supported(int(device), ctypes.byref(out)))
    return bool(out.value)


def flash_attn_uses_mfma(q, k, v, o, p: AttnParams) -> bool:
    """Whether flash_attn runs the MFMA kernel for these arguments (else the general
    kernel); a diagnostic query with no counterpart in the reference."""
    c = p.c()
    res = ctypes.c_int(0)
    _lib.check(_lib.load().mx_flash_attn_uses_mfma(_addr(q), _addr(k), _addr(v), _addr(o), ctypes.byref(c),
                                                   ctypes.byref(res)))
    return bool(res.value)


def flash_attn_split_plan(p: AttnParams, cus: int = 0) -> tuple:
    """(full, units, parts): how flash_attn splits this shape's grid on a device with
    `cus` compute units (0: the current device); a diagnostic query with no counterpart
    in the reference."""
    c = p.c()
    f, u, s = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
    _lib.check(_lib.load().mx_flash_attn_split_plan(ctypes.byref(c), int(cus), ctypes.byref(f), ctypes.byref(u),
                                                    ctypes.byref(s)))
    return f.value, u.value, s.value


def flash_attn_fp8_ok(q, k, v, o, p: AttnParams) -> bool:
    """Reference mx::flash_attn_fp8_ok (src/kernels/attention_fp8.cu:484-486)."""
    c = p.c()
    out = ctypes.c_int(0)
    _lib.check(_lib.load().mx_flash_attn_fp8_ok(_addr(q), _addr(k), _addr(v), _addr(o), ctypes.byref(c),
                                                ctypes.byref(out)))
    return bool(out.value)


def flash_attn_fp8(q, k, v, o, p: AttnParams, ws, stream=None) -> None:
    """Reference mx::flash_attn_fp8 (src/kernels/attention_fp8.cu:488-500)."""
    c = p.c()
    _lib.check(_lib.load().mx_flash_attn_fp8(_addr(q), _addr(k), _addr(v), _addr(o), ctypes.byref(c),
                                             _addr(ws), _stream(stream)))


def sage_layout(p: AttnParams) -> dict:
    c = p.c()
    out = _lib.CLayout()
    _lib.check(_lib.load().mx_sage_layout_of(ctypes.byref(c), ctypes.byref(out)))
    return {name: int(getattr(out, name)) for name, _ in _lib.CLayout._fields_}


def sage_quantize(q, k, v, p: AttnParams, ws, stream=None, q_group: int = 16) -> None:
    """First half of flash_attn_fp8: the Q/K/V quantize prologue into ws. q_group 16 is
    the reference's Q scale grouping; 64 = one Q scale per 64-token block."""
    c = p.c()
    if q_group == 16:
        _lib.check(_lib.load().mx_sage_quantize(_addr(q), _addr(k), _addr(v), ctypes.byref(c), _addr(ws),
                                                _stream(stream)))
    else:
        _lib.check(_lib.load().mx_sage_quantize_qgroup(_addr(q), _addr(k), _addr(v), ctypes.byref(c), _addr(ws),
                                                       int(q_group), _stream(stream)))


def sage_attend(o, p: AttnParams, ws, stream=None) -> None:
    """Second half of flash_attn_fp8: the INT8/FP8 attention kernel on a quantized ws."""
    c = p.c()
    _lib.check(_lib.load().mx_sage_attend(_addr(o), ctypes.byref(c), _addr(ws), _stream(stream)))


ROPE_NONE, ROPE_INTERLEAVED, ROPE_HALF = 0, 1, 2  # reference RopeMode, src/kernels/ops.h:35


def head_norm_rope(inp, S: int, in_stride: int, col0: int, H: int, D: int, norm_w, eps: float, cos, sin,
                   rot: int, mode: int, out, stream=None) -> None:
    """Reference mx::head_norm_rope (src/kernels/ops.h:37-41, ops.cu:197-210): per-head
    RMS-norm (norm_w fp32 [D] or None) then RoPE of the first `rot` channels with
    cos/sin fp32 [S, rot/2]; reads in[s*in_stride + col0 + h*D + d], writes dense
    out [S, H, D] bf16."""
    _lib.check(_lib.load().mx_head_norm_rope(_addr(inp), S, in_stride, col0, H, D, _addr(norm_w), eps,
                                             _addr(cos), _addr(sin), rot, mode, _addr(out), _stream(stream)))


def _norm_rope(q_norm, k_norm, eps, cos, sin, rot, mode):
    return _lib.CNormRope(_addr(q_norm), _addr(k_norm), eps, _addr(cos), _addr(sin), rot, mode)


def sage_quantize_norm_rope(q, k, v, p: AttnParams, q_norm, k_norm, eps: float, cos, sin, rot: int, mode: int,
                            ws, stream=None) -> None:
    """head_norm_rope(q), head_norm_rope(k) and the Sage prologue in one pass: q and k are
    the raw projections (p's strides), q_norm/k_norm fp32 [D] or None, cos/sin fp32
    [rows, rot/2] indexed by token. The workspace equals head_norm_rope + sage_quantize's."""
    c, n = p.c(), _norm_rope(q_norm, k_norm, eps, cos, sin, rot, mode)
    _lib.check(_lib.load().mx_sage_quantize_norm_rope(_addr(q), _addr(k), _addr(v), ctypes.byref(c),
                                                      ctypes.byref(n), _addr(ws), _stream(stream)))


def flash_attn_fp8_norm_rope(q, k, v, o, p: AttnParams, q_norm, k_norm, eps: float, cos, sin, rot: int,
                             mode: int, ws, stream=None) -> None:
    """sage_quantize_norm_rope then the Sage attention kernel (no fallback path)."""
    c, n = p.c(), _norm_rope(q_norm, k_norm, eps, cos, sin, rot, mode)
    _lib.check(_lib.load().mx_flash_attn_fp8_norm_rope(_addr(q), _addr(k), _addr(v), _addr(o), ctypes.byref(c),
                                                       ctypes.byref(n), _addr(ws), _stream(stream)))


def version() -> str:
    return _lib.load().mx_version().decode()

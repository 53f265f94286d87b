"""Host-side mirror of the reference block-scaled GEMM API (src/kernels/blockscale.h:12-37).

QMode / QMat / qmode_name / parse_qmode / qmode_supported / qdata_bytes / qscale_bytes /
quantize_blockscaled / gemm_blockscaled with the reference's names, argument meaning and
errors (RuntimeError for its MX_CHECK). MXFP8 runs on gfx950's scaled MFMA; NVFP4 (e2m1
with e4m3 scales per 16 and a per-tensor amax) is dequantized exactly to f16 inside the
GEMM and runs on the f16 MFMA.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from enum import IntEnum

from . import _lib
from .attention import _addr, _stream


class QMode(IntEnum):
    """Reference QMode (blockscale.h:13)."""
    BF16 = 0
    MXFP8 = 1
    NVFP4 = 2


def qmode_name(m: QMode) -> str:
    """Reference qmode_name (blockscale.cu:9-11)."""
    return "fp4" if m == QMode.NVFP4 else "fp8" if m == QMode.MXFP8 else "bf16"


def parse_qmode(s: str) -> QMode:
    """Reference parse_qmode (blockscale.cu:13-18)."""
    if s in ("fp4", "nvfp4"):
        return QMode.NVFP4
    if s in ("fp8", "mxfp8"):
        return QMode.MXFP8
    if s not in ("bf16", ""):
        raise RuntimeError(f"unknown compute precision {s} (use bf16 / fp8 / fp4)")
    return QMode.BF16


def qmode_supported(m: QMode, device: int = 0) -> bool:
    out = ctypes.c_int(0)
    _lib.check(_lib.load().mx_qmode_supported(int(m), device, ctypes.byref(out)))
    return bool(out.value)


def qdata_bytes(m: QMode, rows: int, K: int) -> int:
    return int(_lib.load().mx_qdata_bytes(int(m), rows, K))


def qscale_bytes(m: QMode, rows: int, K: int) -> int:
    return int(_lib.load().mx_qscale_bytes(int(m), rows, K))


@dataclass
class QMat:
    """Reference QMat (blockscale.h:22-26): quantized data, block scales, (NVFP4) amax."""
    q: object = None
    sf: object = None
    amax: object = None


def quantize_blockscaled(m: QMode, x, ldx: int, rows: int, K: int, out: QMat, stream=None) -> None:
    """Reference quantize_blockscaled (blockscale.cu:113-131)."""
    _lib.check(_lib.load().mx_quantize_blockscaled(int(m), _addr(x), ldx, rows, K, _addr(out.q), _addr(out.sf),
                                                   _addr(out.amax), _stream(stream)))


def gemm_blockscaled(m: QMode, W: QMat, X: QMat, Y, ldy: int, M: int, N: int, K: int, beta: float = 0.0,
                     stream=None) -> None:
    """Reference gemm_blockscaled (blockscale.cu:134-216): Y[M, N] = X W^T (+ Y if beta == 1)."""
    _lib.check(_lib.load().mx_gemm_blockscaled(int(m), _addr(W.q), _addr(W.sf), _addr(W.amax), _addr(X.q),
                                               _addr(X.sf), _addr(X.amax), _addr(Y), ldy, M, N, K, beta,
                                               _stream(stream)))

"""Comparison helpers shared by the parity tests."""
from __future__ import annotations

import numpy as np


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel(); b = np.asarray(b, np.float64).ravel()
    return float(a @ b / max(np.linalg.norm(a) * np.linalg.norm(b), 1e-300))


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def rel_rms(a, ref) -> float:
    a = np.asarray(a, np.float64); ref = np.asarray(ref, np.float64)
    return float(np.sqrt(np.sum((a - ref) ** 2) / max(np.sum(ref ** 2), 1e-30)))


def reference_gate(actual, expected):
    """The reference's flash-vs-reference gate (tests/attention_test.cu:100-116):
    max-abs <= 0.01*max(1, max|ref|) and rel-RMS < 0.01. Returns (ok, max_abs, limit, rel_rms)."""
    a = np.asarray(actual, np.float64); b = np.asarray(expected, np.float64)
    assert np.all(np.isfinite(a)) and np.all(np.isfinite(b)), "nonfinite output"
    err = float(np.max(np.abs(a - b))) if a.size else 0.0
    tol = 0.01 * max(1.0, float(np.max(np.abs(b))) if b.size else 0.0)
    rr = rel_rms(a, b)
    return err <= tol and rr < 0.01, err, tol, rr


def query_rows(sq: int, hq: int):
    """Reference sampled-row rule (tests/attention_test.cu:51-62)."""
    if sq <= 129 or (sq <= 1000 and hq <= 4):
        return list(range(sq))
    return sorted({i for i in (0, 1, 16, 17, 63, 64, 127, 128, sq // 2, sq - 2, sq - 1) if i < sq})

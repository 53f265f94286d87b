"""GPU parity of the MXFP8 and NVFP4 block-scaled quantizers and GEMMs (mx_quantize_blockscaled /
mx_gemm_blockscaled through the C ABI) against the oracle's restatement of the
reference (src/kernels/blockscale.cu:69-108 quantizer, :134-216 GEMM contract):
quantized bytes and scales bit-exact, the GEMM within bf16 rounding of the float64
product of the dequantized operands."""
import numpy as np
import pytest
import torch

import oracle
from miroxen_amd.blockscale import (QMat, QMode, gemm_blockscaled, qdata_bytes, qmode_supported, qscale_bytes,
                                    quantize_blockscaled)

pytestmark = pytest.mark.gpu


def _quant(x, rows, K, cuda, ldx=None):
    ldx = ldx or K
    q = torch.zeros(qdata_bytes(QMode.MXFP8, rows, K) + 64, dtype=torch.uint8, device=cuda)
    sf = torch.full((qscale_bytes(QMode.MXFP8, rows, K),), 0xFF, dtype=torch.uint8, device=cuda)
    quantize_blockscaled(QMode.MXFP8, x, ldx, rows, K, QMat(q, sf))
    return q, sf


def _sf_view(sf, rows, K):
    return oracle.mx_scale_unpack(sf.cpu().numpy(), rows, K)


def test_modes(cuda):
    assert qmode_supported(QMode.BF16) and qmode_supported(QMode.MXFP8) and qmode_supported(QMode.NVFP4)


@pytest.mark.parametrize("rows,K,pad", [(1, 32, 0), (300, 256, 8), (129, 4096, 0), (2048, 3072, 0)])
def test_quantizer_bit_exact(cuda, rows, K, pad):
    print(f"mxfp8 quant rows={rows} K={K} pad={pad}", flush=True)
    rng = np.random.default_rng(rows + K)
    ldx = K + pad
    xf = (rng.standard_normal((rows, ldx)) * np.exp2(rng.integers(-12, 12, (rows, 1)))).astype(np.float32)
    xf[0, :32] = 0.0
    xb = oracle.f32_to_bf16(xf)
    x = torch.from_numpy(xb.view(np.int16)).to(cuda)
    q, sf = _quant(x, rows, K, cuda, ldx)
    torch.cuda.synchronize()
    wq, ws = oracle.mxfp8_quantize(xb, rows, K, ldx)
    assert np.array_equal(q.cpu().numpy()[: rows * K].reshape(rows, K), wq)
    assert np.array_equal(_sf_view(sf, rows, K), ws)
    assert np.all(q.cpu().numpy()[rows * K:] == 0), "wrote past the data"
    # the whole buffer is the reference's interleaved layout of the scales, and padding
    # positions hold 1.0 (127), so padded blocks contribute 0 x 1 in the GEMM
    np.testing.assert_array_equal(sf.cpu().numpy(), oracle.mx_scale_pack(ws, rows, K))


@pytest.mark.parametrize("M,N,K,beta", [
    (256, 256, 128, 0.0), (300, 200, 96, 0.0), (77, 513, 4096, 1.0), (1024, 768, 3072, 0.0), (33, 31, 160, 1.0),
    (512, 512, 256, 1.0),  # beta = 1 on the aligned (16-byte store) path: ldy = N + 8
    (1, 1, 32, 0.0), (1, 300, 64, 1.0),  # the smallest shapes: one row, one column, one K block
])
def test_gemm_matches_oracle(cuda, M, N, K, beta):
    print(f"mxfp8 gemm M={M} N={N} K={K} beta={beta}", flush=True)
    rng = np.random.default_rng(M * 7 + N + K)
    xb = oracle.f32_to_bf16((rng.standard_normal((M, K)) * 2).astype(np.float32))
    wb = oracle.f32_to_bf16((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
    to = lambda a: torch.from_numpy(a.view(np.int16)).to(cuda)
    xq, xs = _quant(to(xb), M, K, cuda)
    wq, ws = _quant(to(wb), N, K, cuda)
    ldy = N + 8
    y0 = oracle.f32_to_bf16(rng.standard_normal((M, ldy)).astype(np.float32))
    y = to(y0).clone()
    gemm_blockscaled(QMode.MXFP8, QMat(wq, ws), QMat(xq, xs), y, ldy, M, N, K, beta)
    torch.cuda.synchronize()
    got = oracle.bf16_to_f32(y.cpu().numpy().view(np.uint16)).astype(np.float64)
    oq, os_ = oracle.mxfp8_quantize(xb, M, K)
    owq, ows = oracle.mxfp8_quantize(wb, N, K)
    want = oracle.gemm_mxfp8(owq, ows, oq, os_, M, N, K).astype(np.float64)
    if beta:
        want = want + oracle.bf16_to_f32(y0)[:, :N].astype(np.float64)
    g = got[:, :N]
    # fp32 accumulation then one bf16 rounding (plus the bf16 of Y for beta = 1)
    tol = np.abs(want) * 2.0 ** -7 + np.abs(want).max() * 2.0 ** -14
    assert np.all(np.abs(g - want) <= tol), float(np.max(np.abs(g - want) - tol))
    np.testing.assert_array_equal(got[:, N:], oracle.bf16_to_f32(y0)[:, N:])  # columns past N untouched


@pytest.mark.parametrize("M,N,K", [(300, 512, 1024), (129, 384, 4160)])
def test_reference_cases_and_gates(cuda, M, N, K):
    """The reference's own cases (tests/blockscale_test.cpp:135-136: M not a multiple of 128;
    K/32 not a multiple of 4) with its generator shape (N(0,1) activations with 1-in-50
    outliers x20, N(0, 0.02) weights, :66-69) and its gates (:93-96): the GEMM equals the
    f32 GEMM of the decoded operands (layout error < 5e-3, here bf16 rounding), the
    activations' element error < 4 %, and the GEMM error against the bf16 GEMM < 5 %."""
    print(f"mxfp8 reference case M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(7 + M)
    xf = rng.standard_normal((M, K)).astype(np.float32)
    xf *= np.where(rng.integers(0, 50, (M, K)) == 0, 20.0, 1.0).astype(np.float32)
    wf = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    xb, wb = oracle.f32_to_bf16(xf), oracle.f32_to_bf16(wf)
    to = lambda a: torch.from_numpy(a.view(np.int16)).to(cuda)
    xq, xs = _quant(to(xb), M, K, cuda)
    wq, ws = _quant(to(wb), N, K, cuda)
    y = torch.zeros(M, N, dtype=torch.bfloat16, device=cuda)
    gemm_blockscaled(QMode.MXFP8, QMat(wq, ws), QMat(xq, xs), y, N, M, N, K)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy().astype(np.float64)
    t = np.array([oracle.e4m3_to_f32(c) for c in range(256)], np.float64)
    dec = lambda q, s, r: (t[q.cpu().numpy()[: r * K].reshape(r, K // 32, 32)] *
                           np.exp2(_sf_view(s, r, K).astype(np.float64) - 127)[..., None]).reshape(r, K)
    fx, fw = dec(xq, xs, M), dec(wq, ws, N)
    ydec = fx @ fw.T
    x64, w64 = oracle.bf16_to_f32(xb).astype(np.float64), oracle.bf16_to_f32(wb).astype(np.float64)
    rel = lambda a, b: float(np.sqrt(((a - b) ** 2).sum() / (b ** 2).sum()))
    layout_err, elem_err, quant_err = rel(got, ydec), rel(fx, x64), rel(got, x64 @ w64.T)
    print(f"layout {layout_err:.2e} element {elem_err:.4f} gemm-vs-bf16 {quant_err:.4f}", flush=True)
    assert layout_err < 5e-3 and elem_err < 0.04 and quant_err < 0.05


def test_gemm_full_size_sampled_rows(cuda):
    """The reference's quoted shape (M=8192, N=12288, K=4096) through the full grid: both
    quantized operands bit-exact against the oracle quantizer, then nine output rows
    spread over every tile row (first, last, tile edges) against the oracle GEMM of
    those rows of X with all of W."""
    M, N, K = 8192, 12288, 4096
    print(f"mxfp8 full-size M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(53)
    x = (torch.randn(M, K, device=cuda, generator=g) * 2).to(torch.bfloat16)
    w = (torch.randn(N, K, device=cuda, generator=g) * 0.05).to(torch.bfloat16)
    xq, xs = _quant(x, M, K, cuda)
    wq, ws = _quant(w, N, K, cuda)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=cuda)
    gemm_blockscaled(QMode.MXFP8, QMat(wq, ws), QMat(xq, xs), y, N, M, N, K)
    torch.cuda.synchronize()
    bits = lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16)
    owq, ows = oracle.mxfp8_quantize(bits(w), N, K)
    assert np.array_equal(wq.cpu().numpy()[: N * K].reshape(N, K), owq)
    assert np.array_equal(_sf_view(ws, N, K), ows)
    rows = np.array([0, 1, 255, 256, 2047, 4100, 6143, 8190, 8191])
    xb = bits(x)[rows]
    oxq, oxs = oracle.mxfp8_quantize(xb, len(rows), K)
    assert np.array_equal(xq.cpu().numpy()[: M * K].reshape(M, K)[rows], oxq)
    assert np.array_equal(_sf_view(xs, M, K)[rows], oxs)
    want = oracle.gemm_mxfp8(owq, ows, oxq, oxs, len(rows), N, K).astype(np.float64)
    got = y.float().cpu().numpy()[rows].astype(np.float64)
    tol = np.abs(want) * 2.0 ** -7 + np.abs(want).max() * 2.0 ** -14
    assert np.all(np.abs(got - want) <= tol), float(np.max(np.abs(got - want) - tol))


# ---------------- NVFP4 (reference blockscale.cu NVFP4 branch) ----------------

def _quant4(x, rows, K, cuda, ldx=None):
    ldx = ldx or K
    q = torch.full((qdata_bytes(QMode.NVFP4, rows, K) + 64,), 0x5A, dtype=torch.uint8, device=cuda)
    sf = torch.full((qscale_bytes(QMode.NVFP4, rows, K),), 0xFF, dtype=torch.uint8, device=cuda)
    am = torch.full((4,), -1.0, dtype=torch.float32, device=cuda)
    quantize_blockscaled(QMode.NVFP4, x, ldx, rows, K, QMat(q, sf, am))
    return q, sf, am


@pytest.mark.parametrize("rows,K,pad", [(1, 32, 0), (300, 512, 8), (129, 4160, 0), (2048, 3072, 0)])
def test_nvfp4_quantizer_bit_exact(cuda, rows, K, pad):
    print(f"nvfp4 quant rows={rows} K={K} pad={pad}", flush=True)
    rng = np.random.default_rng(rows * 3 + K)
    ldx = K + pad
    xf = (rng.standard_normal((rows, ldx)) * np.exp2(rng.integers(-8, 8, (rows, 1)))).astype(np.float32)
    xf[0, :16] = 0.0
    xb = oracle.f32_to_bf16(xf)
    x = torch.from_numpy(xb.view(np.int16)).to(cuda)
    q, sf, am = _quant4(x, rows, K, cuda, ldx)
    torch.cuda.synchronize()
    wq, ws, wa = oracle.nvfp4_quantize(xb, rows, K, ldx)
    qh = q.cpu().numpy()
    assert float(am[0]) == wa
    assert np.array_equal(qh[: rows * K // 2].reshape(rows, K // 2), wq)
    assert np.all(qh[rows * K // 2:] == 0x5A), "wrote past the data"
    # the whole scale buffer: the reference's interleave of the e4m3 scales, padding 0
    np.testing.assert_array_equal(sf.cpu().numpy(), oracle.mx_scale_pack(ws, rows, K, fill=0, vec=16))


@pytest.mark.parametrize("M,N,K,beta", [
    (256, 256, 256, 0.0), (300, 200, 96, 0.0), (77, 513, 4096, 1.0), (1024, 768, 3072, 0.0), (33, 31, 160, 1.0),
    (512, 512, 512, 1.0), (1, 1, 32, 0.0), (1, 300, 64, 1.0),
])
def test_nvfp4_gemm_matches_oracle(cuda, M, N, K, beta):
    print(f"nvfp4 gemm M={M} N={N} K={K} beta={beta}", flush=True)
    rng = np.random.default_rng(M * 5 + N + K)
    xb = oracle.f32_to_bf16((rng.standard_normal((M, K)) * 2).astype(np.float32))
    wb = oracle.f32_to_bf16((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
    to = lambda a: torch.from_numpy(a.view(np.int16)).to(cuda)
    xq, xs, xa = _quant4(to(xb), M, K, cuda)
    wq, ws, wa = _quant4(to(wb), N, K, cuda)
    ldy = N + 8
    y0 = oracle.f32_to_bf16(rng.standard_normal((M, ldy)).astype(np.float32))
    y = to(y0).clone()
    gemm_blockscaled(QMode.NVFP4, QMat(wq, ws, wa), QMat(xq, xs, xa), y, ldy, M, N, K, beta)
    torch.cuda.synchronize()
    got = oracle.bf16_to_f32(y.cpu().numpy().view(np.uint16)).astype(np.float64)
    oq, os_, oa = oracle.nvfp4_quantize(xb, M, K)
    owq, ows, owa = oracle.nvfp4_quantize(wb, N, K)
    want = oracle.gemm_nvfp4(owq, ows, owa, oq, os_, oa, M, N, K).astype(np.float64)
    if beta:
        want = want + oracle.bf16_to_f32(y0)[:, :N].astype(np.float64)
    g = got[:, :N]
    # exact products, fp32 accumulation, alpha in fp32, then one bf16 rounding
    tol = np.abs(want) * 2.0 ** -7 + np.abs(want).max() * 2.0 ** -14
    assert np.all(np.abs(g - want) <= tol), float(np.max(np.abs(g - want) - tol))
    np.testing.assert_array_equal(got[:, N:], oracle.bf16_to_f32(y0)[:, N:])


@pytest.mark.parametrize("M,N,K", [(300, 512, 1024), (129, 384, 4160)])
def test_nvfp4_reference_cases_and_gates(cuda, M, N, K):
    """The reference's NVFP4 cases and gates (tests/blockscale_test.cpp:93-96, :135-136):
    the GEMM equals the f32 GEMM of the operands decoded by the reference test's decoder
    (layout error < 5e-3), the activations' element error < 12 %, and the GEMM error
    against the bf16 GEMM < 15 %."""
    print(f"nvfp4 reference case M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(7 + M)
    xf = rng.standard_normal((M, K)).astype(np.float32)
    xf *= np.where(rng.integers(0, 50, (M, K)) == 0, 20.0, 1.0).astype(np.float32)
    wf = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    xb, wb = oracle.f32_to_bf16(xf), oracle.f32_to_bf16(wf)
    to = lambda a: torch.from_numpy(a.view(np.int16)).to(cuda)
    xq, xs, xa = _quant4(to(xb), M, K, cuda)
    wq, ws, wa = _quant4(to(wb), N, K, cuda)
    y = torch.zeros(M, N, dtype=torch.bfloat16, device=cuda)
    gemm_blockscaled(QMode.NVFP4, QMat(wq, ws, wa), QMat(xq, xs, xa), y, N, M, N, K)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy().astype(np.float64)
    t = np.array([oracle.e4m3_to_f32(c) for c in range(256)], np.float64)
    mag = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float64)

    def dec(q, s, am, r):  # the reference test's decoder (:37-43)
        b = q.cpu().numpy()[: r * K // 2].reshape(r, K // 2)
        codes = np.stack([b & 15, b >> 4], -1).reshape(r, K)
        v = np.where(codes & 8, -1.0, 1.0) * mag[codes & 7]
        g = float(am[0]) / (6 * 448) if float(am[0]) > 0 else 1.0
        sc = t[oracle.mx_scale_unpack(s.cpu().numpy(), r, K, vec=16)] * g
        return (v.reshape(r, K // 16, 16) * sc[..., None]).reshape(r, K)

    fx, fw = dec(xq, xs, xa, M), dec(wq, ws, wa, N)
    ydec = fx @ fw.T
    x64, w64 = oracle.bf16_to_f32(xb).astype(np.float64), oracle.bf16_to_f32(wb).astype(np.float64)
    rel = lambda a, b: float(np.sqrt(((a - b) ** 2).sum() / (b ** 2).sum()))
    layout_err, elem_err, quant_err = rel(got, ydec), rel(fx, x64), rel(got, x64 @ w64.T)
    print(f"nvfp4 layout {layout_err:.2e} element {elem_err:.4f} gemm-vs-bf16 {quant_err:.4f}", flush=True)
    assert layout_err < 5e-3 and elem_err < 0.12 and quant_err < 0.15


def test_nvfp4_gemm_full_size_sampled_rows(cuda):
    """NVFP4 at the reference's quoted shape (M=8192, N=12288, K=4096) through the full
    grid: W's quantization bit-exact against the oracle, then nine output rows spread
    over every tile row against the oracle GEMM of those rows (with X's amax, which the
    oracle recomputes over the sampled rows only, replaced by the device's)."""
    M, N, K = 8192, 12288, 4096
    print(f"nvfp4 full-size M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(57)
    x = (torch.randn(M, K, device=cuda, generator=g) * 2).to(torch.bfloat16)
    w = (torch.randn(N, K, device=cuda, generator=g) * 0.05).to(torch.bfloat16)
    xq, xs, xa = _quant4(x, M, K, cuda)
    wq, ws, wa = _quant4(w, N, K, cuda)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=cuda)
    gemm_blockscaled(QMode.NVFP4, QMat(wq, ws, wa), QMat(xq, xs, xa), y, N, M, N, K)
    torch.cuda.synchronize()
    bits = lambda t: t.view(torch.int16).cpu().numpy().view(np.uint16)
    owq, ows, owa = oracle.nvfp4_quantize(bits(w), N, K)
    assert float(wa[0]) == owa
    assert np.array_equal(wq.cpu().numpy()[: N * K // 2].reshape(N, K // 2), owq)
    assert np.array_equal(oracle.mx_scale_unpack(ws.cpu().numpy(), N, K, vec=16), ows)
    rows = np.array([0, 1, 255, 256, 2047, 4100, 6143, 8190, 8191])
    xqh = xq.cpu().numpy()[: M * K // 2].reshape(M, K // 2)[rows]
    xsh = oracle.mx_scale_unpack(xs.cpu().numpy(), M, K, vec=16)[rows]
    want = oracle.gemm_nvfp4(owq, ows, owa, xqh, xsh, float(xa[0]), len(rows), N, K).astype(np.float64)
    got = y.float().cpu().numpy()[rows].astype(np.float64)
    tol = np.abs(want) * 2.0 ** -7 + np.abs(want).max() * 2.0 ** -14
    assert np.all(np.abs(got - want) <= tol), float(np.max(np.abs(got - want) - tol))

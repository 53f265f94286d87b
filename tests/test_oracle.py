"""Pins the CPU oracle (oracle/oracle.c) against facts that do not come from its
own formulas: the OCP FP8 table and nearest-value search, torch's bf16 rounding,
a numpy float64 attention, closed-form special cases and invariants."""
import numpy as np
import pytest
import torch

import oracle
from tests.helpers import cosine, rel_rms


# ---------------- e4m3 (OCP FP8 E4M3FN) ----------------

def _e4m3_table():
    """Decode table straight from the OCP spec: e=0 subnormal m*2^-9, else (1+m/8)*2^(e-7);
    S.1111.111 is NaN."""
    vals = {}
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            continue
        v = m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
        vals[c] = -v if s else v
    return vals


def test_e4m3_decode_matches_spec_table():
    for c, v in _e4m3_table().items():
        assert oracle.e4m3_to_f32(c) == v, hex(c)
    assert np.isnan(oracle.e4m3_to_f32(0x7F)) and np.isnan(oracle.e4m3_to_f32(0xFF))
    assert max(_e4m3_table().values()) == 448.0


def test_e4m3_roundtrip_all_codes():
    for c, v in _e4m3_table().items():
        assert oracle.e4m3(v) == c, (hex(c), v)


def test_e4m3_is_nearest_even_by_search():
    table = _e4m3_table()
    codes = np.array([c for c in table if c != 0x80])  # +0 represents zero
    vals = np.array([table[c] for c in codes])
    rng = np.random.default_rng(7)
    xs = np.concatenate([rng.uniform(-460, 460, 3000), rng.uniform(-0.03, 0.03, 2000),
                         (vals[:-1] + np.diff(vals) / 2)[np.diff(vals) > 0]])  # all midpoints
    for x in xs.astype(np.float32):
        x = float(x)
        d = np.abs(vals - x)
        best = np.flatnonzero(d == d.min())
        if len(best) > 1:  # tie: the even code (mantissa lsb 0) wins
            best = [b for b in best if codes[b] & 1 == 0]
        want = int(codes[best[0]])
        if want == 0 and np.signbit(x):
            want = 0x80
        assert oracle.e4m3(x) == want, (x, hex(oracle.e4m3(x)), hex(want))


def test_e4m3_saturates_and_subnormals():
    assert oracle.e4m3(448.0) == 0x7E and oracle.e4m3(1e6) == 0x7E and oracle.e4m3(-1e6) == 0xFE
    assert oracle.e4m3(470.0) == 0x7E  # SATFINITE, not NaN
    assert oracle.e4m3(2.0 ** -9) == 0x01 and oracle.e4m3(2.0 ** -10) == 0x00  # tie -> even (0)
    assert oracle.e4m3(1.5 * 2.0 ** -9) == 0x02  # tie between 1 and 2 -> even (2)
    assert oracle.e4m3(1.0) == 0x38 and oracle.e4m3(-2.0) == 0xC0


# ---------------- bf16 ----------------

def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10,
                        # exact ties: low 16 bits = 0x8000
                        (rng.integers(0, 2 ** 16, 1000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)])
    x = x[np.isfinite(x)]
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16(x), want)
    lib = oracle.lib()
    for xv in x[:200]:
        assert lib.or_f32_to_bf16(float(xv)) == oracle.f32_to_bf16(np.array([xv]))[0]


# ---------------- exact attention ----------------

def _np_attention(q, k, v, Hq, Hkv, D, scale, causal=0, q_offset=0, mask=None):
    """Independent float64 attention with numpy (q [Sq,Hq,D], k/v [Skv,Hkv,D] float)."""
    Sq, Skv = q.shape[0], k.shape[0]
    out = np.zeros((Sq, Hq, D))
    g = Hq // Hkv
    for h in range(Hq):
        s = q[:, h, :] @ k[:, h // g, :].T * scale
        live = np.ones((Sq, Skv), bool)
        if mask is not None:
            live &= mask[None, :].astype(bool)
        if causal:
            live &= np.arange(Skv)[None, :] <= (q_offset + np.arange(Sq))[:, None]
        s = np.where(live, s, -np.inf)
        mx = s.max(1, keepdims=True)
        mx = np.where(np.isfinite(mx), mx, 0)
        w = np.where(live, np.exp(s - mx), 0)
        den = w.sum(1, keepdims=True)
        out[:, h, :] = np.where(den > 0, (w @ v[:, h // g, :]) / np.where(den > 0, den, 1), 0)
    return out


def _bf16_rand(rng, shape, mag=1.0):
    return oracle.f32_to_bf16(rng.standard_normal(shape).astype(np.float32) * mag)


@pytest.mark.parametrize("Sq,Skv,Hq,Hkv,D,causal,off,scale,masked", [
    (7, 13, 2, 1, 64, 0, 0, 0.0, False),
    (5, 40, 4, 2, 72, 1, 3, 0.0, False),
    (9, 33, 2, 2, 128, 0, 0, -0.125, True),
    (17, 65, 3, 1, 128, 1, -2, 0.3, True),
])
def test_attention_f64_matches_numpy(Sq, Skv, Hq, Hkv, D, causal, off, scale, masked):
    rng = np.random.default_rng(Sq * 100 + Skv)
    q = _bf16_rand(rng, (Sq, Hq, D), 2.0); k = _bf16_rand(rng, (Skv, Hkv, D), 2.0)
    v = _bf16_rand(rng, (Skv, Hkv, D))
    mask = (rng.random(Skv) > 0.3).astype(np.uint8) if masked else None
    got = oracle.attention_f64(q, k, v, Sq, Skv, Hq, Hkv, D, scale, causal, off, kv_valid=mask)
    sc = scale if scale != 0 else 1 / np.sqrt(D)
    want = _np_attention(oracle.bf16_to_f32(q).reshape(Sq, Hq, D).astype(np.float64),
                         oracle.bf16_to_f32(k).reshape(Skv, Hkv, D).astype(np.float64),
                         oracle.bf16_to_f32(v).reshape(Skv, Hkv, D).astype(np.float64),
                         Hq, Hkv, D, sc, causal, off, mask)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_attention_f64_strided_rows():
    rng = np.random.default_rng(3)
    Sq, Skv, H, D, pad = 6, 11, 2, 64, 5
    qs, ks = H * D + pad, H * D + pad + 2
    q = _bf16_rand(rng, (Sq, qs)); k = _bf16_rand(rng, (Skv, ks)); v = _bf16_rand(rng, (Skv, ks))
    got = oracle.attention_f64(q, k, v, Sq, Skv, H, H, D, q_stride=qs, kv_stride=ks, rows=[0, 3, 5])
    dense = lambda t, S: t[:, : H * D].reshape(S, H * D)
    want = oracle.attention_f64(dense(q, Sq), dense(k, Skv), dense(v, Skv), Sq, Skv, H, H, D, rows=[0, 3, 5])
    np.testing.assert_array_equal(got, want)


def test_attention_uniform_scores_give_mean_of_v():
    rng = np.random.default_rng(4)
    Skv, H, D = 50, 2, 128
    q = np.zeros((3, H, D), np.uint16)  # q = 0 -> all scores equal
    k = _bf16_rand(rng, (Skv, H, D)); v = _bf16_rand(rng, (Skv, H, D))
    mask = np.ones(Skv, np.uint8); mask[::3] = 0
    got = oracle.attention_f64(q, k, v, 3, Skv, H, H, D, kv_valid=mask)
    vf = oracle.bf16_to_f32(v).reshape(Skv, H, D)[mask.astype(bool)].astype(np.float64).mean(0)
    np.testing.assert_allclose(got, np.broadcast_to(vf, got.shape), rtol=1e-6, atol=1e-7)


def test_attention_mask_equals_compacted_keys():
    rng = np.random.default_rng(5)
    Sq, Skv, H, D = 8, 70, 2, 128
    q = _bf16_rand(rng, (Sq, H, D), 3.0); k = _bf16_rand(rng, (Skv, H, D), 3.0); v = _bf16_rand(rng, (Skv, H, D))
    mask = (rng.random(Skv) > 0.4).astype(np.uint8)
    sel = mask.astype(bool)
    a = oracle.attention_f64(q, k, v, Sq, Skv, H, H, D, kv_valid=mask)
    b = oracle.attention_f64(q, k[sel], v[sel], Sq, int(sel.sum()), H, H, D)
    np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)


def test_attention_all_masked_row_is_zero():
    rng = np.random.default_rng(6)
    q = _bf16_rand(rng, (2, 1, 64)); k = _bf16_rand(rng, (5, 1, 64)); v = _bf16_rand(rng, (5, 1, 64))
    got = oracle.attention_f64(q, k, v, 2, 5, 1, 1, 64, kv_valid=np.zeros(5, np.uint8))
    assert np.all(got == 0)


# ---------------- Sage prologue ----------------

def test_quant_rows_hand_vectors():
    D, G = 128, 16
    x = np.zeros((20, 1, D), np.float32)
    x[0, 0, 0] = 127.0          # amax = 127 -> inv = 1
    x[1, 0, :4] = [2.5, 3.5, -2.5, -127.0]   # ties round to even: 2, 4, -2; -amax -> -127
    x[2, 0, 5] = 0.5            # tie -> 0
    # second group (rows 16..19): all zero -> scale 0, q 0; rows >= S (20) padded to 32 -> 0
    q, s = oracle.quant_rows(oracle.f32_to_bf16(x), D, 20, 32, 1, D, G, None, 2.0)
    assert q[0, 0, 0] == 127 and list(q[0, 1, :4]) == [2, 4, -2, -127] and q[0, 2, 5] == 0
    assert np.all(q[0, 16:] == 0)
    assert s[0, 0] == np.float32(127.0) / np.float32(127.0) * np.float32(2.0) and s[0, 1] == 0.0


def test_quant_rows_mean_and_scale_vs_numpy():
    rng = np.random.default_rng(8)
    S, H, D, G = 150, 3, 128, 64
    xb = _bf16_rand(rng, (S, H, D), 3.0)
    mean = rng.standard_normal((H, D)).astype(np.float32)
    q, s = oracle.quant_rows(xb, H * D, S, 192, H, D, G, mean, 1.0)
    xf = oracle.bf16_to_f32(xb).reshape(S, H, D)
    xf = np.concatenate([xf - mean[None], np.zeros((192 - S, H, D), np.float32)]).astype(np.float32)
    xf[S:] = 0
    for h in range(H):
        for g in range(192 // G):
            blk = xf[g * G:(g + 1) * G, h, :]
            am = np.float32(np.abs(blk).max())
            inv = np.float32(127.0) / am if am > 0 else np.float32(0)
            want = np.rint(blk * inv).astype(np.int8)
            assert np.array_equal(q[h, g * G:(g + 1) * G], want)
            assert s[h, g] == np.float32(am / np.float32(127.0) * np.float32(1.0))
    assert np.all(np.abs(q.astype(int)) <= 127)


def test_kv_stats_vs_numpy():
    rng = np.random.default_rng(9)
    for Skv in (200, 700):
        H, D = 2, 128
        k = _bf16_rand(rng, (Skv, H, D), 2.0); v = _bf16_rand(rng, (Skv, H, D))
        km, va = oracle.kv_stats(k, v, Skv, H, D)
        kf = oracle.bf16_to_f32(k).reshape(Skv, H, D); vf = oracle.bf16_to_f32(v).reshape(Skv, H, D)
        want = np.zeros((H, D), np.float32)
        for b in range(0, Skv, 256):
            # np.cumsum in float32 is a sequential left-to-right float sum
            part = np.cumsum(kf[b:b + 256], axis=0, dtype=np.float32)[-1]
            want = (want + part / np.float32(Skv)).astype(np.float32)
        assert np.array_equal(km, want)
        assert np.array_equal(va, np.abs(vf).max(0))
        np.testing.assert_allclose(km, kf.astype(np.float64).mean(0), atol=1e-5)


def test_v_quant_layout_and_values():
    rng = np.random.default_rng(10)
    Skv, H, D = 70, 2, 128
    v = _bf16_rand(rng, (Skv, H, D))
    va = np.abs(oracle.bf16_to_f32(v).reshape(Skv, H, D)).max(0)
    va[1, 7] = 0.0  # a zero channel quantizes to 0
    vt = oracle.v_quant(v, Skv, H, D, H * D, 128, va)
    assert vt.shape == (H, D, 128) and np.all(vt[:, :, Skv:] == 0) and np.all(vt[1, 7] == 0)
    vf = oracle.bf16_to_f32(v).reshape(Skv, H, D)
    for (h, d, key) in [(0, 0, 0), (1, 127, 69), (0, 64, 33)]:
        assert vt[h, d, key] == oracle.e4m3(np.float32(vf[key, h, d]) * (np.float32(448) / va[h, d]))
    # the channel max maps to +-448
    h, d = 0, 5
    key = int(np.argmax(np.abs(vf[:, h, d])))
    assert vt[h, d, key] & 0x7F == 0x7E


# ---------------- Sage emulator ----------------

def test_sage_single_live_key_returns_dequantized_v():
    rng = np.random.default_rng(11)
    Sq, Skv, H, D = 3, 64, 1, 128
    q = _bf16_rand(rng, (Sq, H, D)); k = _bf16_rand(rng, (Skv, H, D)); v = _bf16_rand(rng, (Skv, H, D))
    mask = np.zeros(Skv, np.uint8); mask[37] = 1
    out, t = oracle.sage_reference(q, k, v, Sq, Skv, H, H, D, kv_valid=mask)
    # one live key: P = e4m3(~448) = 448, l ~ 448 (up to the exponent's float rounding in
    # the reference formulation) -> out = e4m3(v*448/a) * a / 448
    deq = np.array([oracle.e4m3_to_f32(c) for c in t["vt"][0, :, 37]], np.float32) * t["va"][0] / np.float32(448)
    np.testing.assert_allclose(out[:, 0, :], np.broadcast_to(deq, (Sq, D)), rtol=1e-4, atol=1e-7)


def test_sage_uniform_scores_give_mean_of_dequantized_v():
    rng = np.random.default_rng(12)
    Sq, Skv, H, D = 2, 100, 1, 128
    q = np.zeros((Sq, H, D), np.uint16)
    k = _bf16_rand(rng, (Skv, H, D)); v = _bf16_rand(rng, (Skv, H, D))
    out, t = oracle.sage_reference(q, k, v, Sq, Skv, H, H, D)
    deq = np.vectorize(oracle.e4m3_to_f32)(t["vt"][0, :, :Skv]).astype(np.float64).mean(1) * t["va"][0] / 448
    np.testing.assert_allclose(out[:, 0, :], np.broadcast_to(deq, (Sq, D)), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("Sq,Skv,Hq,Hkv,kbias,vbias", [
    (300, 300, 4, 4, 0.0, 0.5),    # reference cases tests/attention_fp8_test.cpp:110-113 (scaled)
    (257, 1000, 4, 2, 4.0, 0.5),
    (200, 4352, 1, 1, 8.0, 0.5),
])
def test_sage_emulator_reference_gate(Sq, Skv, Hq, Hkv, kbias, vbias):
    """rel-RMS < 4% against exact attention (tests/attention_fp8_test.cpp:65), with the
    reference's per-channel K bias (and V bias) generator (:18-27)."""
    rng = np.random.default_rng(Sq * 31 + Skv)
    D = 128
    q = _bf16_rand(rng, (Sq, Hq, D))
    kb = rng.standard_normal(Hkv * D).astype(np.float32) * kbias
    vb = rng.standard_normal(Hkv * D).astype(np.float32) * vbias
    k = oracle.f32_to_bf16((rng.standard_normal((Skv, Hkv * D)) + kb).astype(np.float32))
    v = oracle.f32_to_bf16((rng.standard_normal((Skv, Hkv * D)) + vb).astype(np.float32))
    rows = np.arange(0, Sq, 7, dtype=np.int32)
    out, _ = oracle.sage_reference(q, k, v, Sq, Skv, Hq, Hkv, D, rows=rows)
    exact = oracle.attention_f64(q, k, v, Sq, Skv, Hq, Hkv, D, rows=rows)
    assert rel_rms(out, exact) < 0.04
    assert cosine(out, exact) > 0.995


def test_sage_lazy_max_headroom_matches_reference_rule():
    """The kernel's lazy running max (headroom H) vs the reference's exact max (H = 0):
    same quantized inputs, outputs equal up to fp8 rounding of P."""
    rng = np.random.default_rng(13)
    Sq, Skv, H, D = 64, 700, 2, 128
    q = _bf16_rand(rng, (Sq, H, D), 2.0); k = _bf16_rand(rng, (Skv, H, D), 2.0); v = _bf16_rand(rng, (Skv, H, D))
    mask = (rng.random(Skv) > 0.2).astype(np.uint8)
    exact_rule, _ = oracle.sage_reference(q, k, v, Sq, Skv, H, H, D, kv_valid=mask)
    lazy, _ = oracle.sage_reference(q, k, v, Sq, Skv, H, H, D, kv_valid=mask, headroom=oracle.KERNEL_HEADROOM)
    exact = oracle.attention_f64(q, k, v, Sq, Skv, H, H, D, kv_valid=mask)
    # the two rules round P differently; both must be equally close to exact attention
    assert rel_rms(lazy, exact) <= 1.1 * rel_rms(exact_rule, exact) + 1e-3
    assert rel_rms(lazy, exact) < 0.04 and cosine(lazy, exact) > 0.995
    assert cosine(lazy, exact_rule) > 0.999


def _sage_hand_inputs(scores, D=128, seed=21):
    """Quantized Sage operands built by hand so every score is known exactly: one query
    row whose int8 vector is all ones, keys whose channels sum to the integer score (the
    int32 dot product is that integer), Q scale 2^-11 and K scales 1, random e4m3 V codes
    (no NaN code) and per-channel V scales. scores: {key: score in units of 1/16 log2};
    every other key is dead (masked). Returns the emulator's arguments, the mask and
    the dequantized V rows.

    Why sc = 2^-11: the reference's exponent (attention_fp8.cu:331, :337) is one FMA
    with nm = (log2 448 - H - m) - 12582912 sc rounded to a float of magnitude
    12582912 sc = 6144, whose ulp is 2^-11; so every weight carries a relative error
    of at most 2^(2^-12) - 1 = 1.7e-4 and the closed forms hold to 5e-4."""
    rng = np.random.default_rng(seed)
    Skv = (max(scores) // 64 + 1) * 64
    qi = np.zeros((1, 256, D), np.int8); qi[0, 0, :] = 1
    ki = np.zeros((1, Skv, D), np.int8)
    mask = np.zeros(Skv, np.uint8)
    for key, s16 in scores.items():
        s = s16 * 128  # x = s * 2^-11 = s16 / 16
        ki[0, key, :] = s // D
        ki[0, key, : s % D] += 1
        assert int(ki[0, key].astype(np.int64).sum()) == s
        mask[key] = 1
    qs = np.full((1, 16), 2.0 ** -11, np.float32)
    ks = np.ones((1, Skv // 64), np.float32)
    codes = rng.integers(0, 0x7E, (1, D, Skv)) | (rng.integers(0, 2, (1, D, Skv)) << 7)
    vt = codes.astype(np.uint8)
    va = rng.uniform(0.5, 2.0, (1, D)).astype(np.float32)
    table = _e4m3_table()
    vhat = {key: np.array([table[int(c)] for c in vt[0, :, key]]) for key in scores}
    args = (qi, ki, vt, qs, ks, va, 1, Skv, 1, 1, D)
    return args, mask, vhat, va[0].astype(np.float64)


@pytest.mark.parametrize("headroom,p_live2", [(0.0, 352.0), (3.0, 44.0)])
def test_sage_two_live_keys_closed_form(headroom, p_live2):
    """Two live keys in one tile, scores 10 and 5 (x = s / 16, gap 5/16 in log2 units).
    The running max is the larger score, so P_0 = 448 * 2^-H exactly and the second
    weight is f = 448 * 2^-H * 2^-(5/16) = 360.73 (H = 0) or 45.09 (H = 3), which is not
    an e4m3 value: P_1 = e4m3(f) = 352 or 44 (hand-rounded from the OCP grid). The
    reference accumulates rounded P into O (attention_fp8.cu:352) but sums the
    UNROUNDED f into l (:339, :345) and divides by 448 l in the epilogue (:405-416):
        out[d] = (P_0 v0[d] + P_1 v1[d]) * va[d] / (448 (P_0 + f)).
    A wrong 448 constant, l over rounded P or P left unrounded all miss this by > 1 %."""
    args, mask, vhat, va = _sage_hand_inputs({3: 10, 40: 5})
    out = oracle.sage_emulate(*args, kv_valid=mask, headroom=headroom)[0, 0]
    p0 = 448.0 * 2.0 ** -headroom
    f1 = p0 * 2.0 ** (-5 / 16)
    assert abs(f1 - p_live2) > 1.0  # the second weight really is rounded
    want = (p0 * vhat[3] + p_live2 * vhat[40]) * va / (448.0 * (p0 + f1))
    np.testing.assert_allclose(out, want, rtol=5e-4, atol=1e-6)


@pytest.mark.parametrize("headroom,gap16,rescaled,p_b", [
    (0.0, 40, True, 448.0),    # reference rule: any larger tile max moves m
    (3.0, 56, True, 56.0),     # lazy rule: gap 3.5 > H moves m
    (3.0, 40, False, 320.0),   # lazy rule: gap 2.5 <= H keeps m, P_b = e4m3(56 * 2^2.5)
])
def test_sage_cross_tile_rescale_closed_form(headroom, gap16, rescaled, p_b):
    """Key 0 (tile 0, score 16) and key 64 (tile 1, score 16 + gap16): x_b - x_a = g =
    gap16 / 16 in log2 units. Tile 0 sets m = x_a, P_a = 448 * 2^-H, l = P_a, acc = P_a v_a.
    Tile 1 (attention_fp8.cu:322-353): when m moves to x_b, alpha = 2^-g rescales l and
    acc (:328, :345, :347-353) and P_b = 448 * 2^-H; when the lazy rule keeps m, alpha = 1
    and f_b = 448 * 2^-H * 2^g, rounded to e4m3 in acc but not in l:
        out[d] = (alpha P_a v_a[d] + P_b v_b[d]) * va[d] / (448 (alpha P_a + f_b))."""
    args, mask, vhat, va = _sage_hand_inputs({0: 16, 64: 16 + gap16})
    out = oracle.sage_emulate(*args, kv_valid=mask, headroom=headroom)[0, 0]
    g = gap16 / 16
    pa = 448.0 * 2.0 ** -headroom
    if rescaled:
        alpha, fb = 2.0 ** -g, pa
    else:
        alpha, fb = 1.0, pa * 2.0 ** g
        assert abs(fb - p_b) > 1.0
    want = (alpha * pa * vhat[0] + p_b * vhat[64]) * va / (448.0 * (alpha * pa + fb))
    np.testing.assert_allclose(out, want, rtol=5e-4, atol=1e-6)
    # the same keys in the opposite tile order never rescale: P of the later, smaller
    # key is e4m3(448 * 2^-H * 2^-g), l gets the unrounded weight
    args, mask, vhat, va = _sage_hand_inputs({0: 16 + gap16, 64: 16})
    out = oracle.sage_emulate(*args, kv_valid=mask, headroom=headroom)[0, 0]
    f_small = pa * 2.0 ** -g
    p_small = _e4m3_table()[oracle.e4m3(np.float32(f_small))]
    want = (pa * vhat[0] + p_small * vhat[64]) * va / (448.0 * (pa + f_small))
    np.testing.assert_allclose(out, want, rtol=5e-4, atol=1e-6)


# ---------------- head_norm_rope (reference src/kernels/ops.cu:87-119) ----------------

def _nr_inputs(S, H, D, seed, stride_extra=0, col0=0):
    rng = np.random.default_rng(seed)
    stride = col0 + H * D + stride_extra
    x = oracle.f32_to_bf16((rng.standard_normal((S, stride)) * 1.7).astype(np.float32))
    return x, stride


def _ulps(a, b):
    """bf16 ulp distance of two bf16 bit arrays (same sign assumed for non-zero)."""
    fa, fb = oracle.bf16_to_f32(a).astype(np.float64), oracle.bf16_to_f32(b).astype(np.float64)
    ulp = np.maximum(np.abs(fb), 1e-30) * 2.0 ** -7
    return np.abs(fa - fb) / ulp


def test_head_norm_rope_identity():
    """No norm and rot = 0: a strided gather, bit-exact."""
    S, H, D, col0 = 5, 3, 72, 16
    x, stride = _nr_inputs(S, H, D, 1, stride_extra=8, col0=col0)
    out = oracle.head_norm_rope(x, S, stride, col0, H, D)
    want = x[:, col0:col0 + H * D].reshape(S, H, D)
    assert np.array_equal(out, want)


@pytest.mark.parametrize("D", [64, 72, 128, 256])
def test_head_norm_rope_norm_matches_float64(D):
    S, H = 7, 2
    x, stride = _nr_inputs(S, H, D, D)
    w = np.random.default_rng(3).uniform(0.5, 1.5, D).astype(np.float32)
    eps = 1e-6
    out = oracle.head_norm_rope(x, S, stride, 0, H, D, norm_w=w, eps=eps)
    xf = oracle.bf16_to_f32(x).astype(np.float64).reshape(S, H, D)
    want = xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + eps) * w
    got = oracle.bf16_to_f32(out).astype(np.float64)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-3)) <= 2.0 ** -7  # within bf16 rounding


@pytest.mark.parametrize("mode", [1, 2])
def test_head_norm_rope_rope_is_complex_rotation(mode):
    S, H, D, rot = 6, 2, 128, 96
    x, stride = _nr_inputs(S, H, D, 11)
    rng = np.random.default_rng(5)
    ang = rng.uniform(-np.pi, np.pi, (S, rot // 2))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    out = oracle.bf16_to_f32(oracle.head_norm_rope(x, S, stride, 0, H, D, cos=cs, sin=sn, rot=rot, mode=mode))
    xf = oracle.bf16_to_f32(x).astype(np.float64).reshape(S, H, D)
    half = rot // 2
    if mode == 1:
        a, b = xf[..., 0:rot:2], xf[..., 1:rot:2]
    else:
        a, b = xf[..., :half], xf[..., half:rot]
    z = (a + 1j * b) * np.exp(1j * ang.astype(np.float64))[:, None, :]
    if mode == 1:
        ga, gb = out[..., 0:rot:2], out[..., 1:rot:2]
    else:
        ga, gb = out[..., :half], out[..., half:rot]
    tol = 2.0 ** -8 * (np.abs(z) + 1e-3)
    assert np.all(np.abs(ga - z.real) <= tol) and np.all(np.abs(gb - z.imag) <= tol)
    assert np.array_equal(out[..., rot:], xf[..., rot:].astype(np.float32))  # untouched tail


def test_head_norm_rope_half_equals_permuted_interleaved():
    """ROPE_HALF on channels (i, i+rot/2) == ROPE_INTERLEAVED on the same values laid out
    as (2i, 2i+1), bit for bit (no norm: the rotation alone)."""
    S, H, D = 4, 3, 64
    x, stride = _nr_inputs(S, H, D, 21)
    ang = np.random.default_rng(8).uniform(-3, 3, (S, D // 2))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    perm = np.empty(D, np.int64)
    perm[0::2], perm[1::2] = np.arange(D // 2), np.arange(D // 2, D)
    xi = x.reshape(S, H, D)[..., perm].reshape(S, H * D)
    half = oracle.head_norm_rope(x, S, stride, 0, H, D, cos=cs, sin=sn, rot=D, mode=2)
    inter = oracle.head_norm_rope(xi, S, H * D, 0, H, D, cos=cs, sin=sn, rot=D, mode=1)
    assert np.array_equal(inter, half[..., perm])


def _shfl_xor_block_sum(vals, D):
    """The reference's block_sum (ops.cu:14-29) simulated lane by lane in float32:
    __shfl_xor_sync butterflies within 32-thread warps, then over the warp partials."""
    nthreads = (D + 31) // 32 * 32
    v = np.zeros(nthreads, np.float32); v[:D] = vals
    for o in (16, 8, 4, 2, 1):
        v = (v + v[np.arange(nthreads) ^ o]).astype(np.float32)
    sh = np.zeros(32, np.float32); sh[: nthreads // 32] = v[::32]
    for o in (16, 8, 4, 2, 1):
        sh = (sh + sh[np.arange(32) ^ o]).astype(np.float32)
    return sh[0]


@pytest.mark.parametrize("D", [64, 72, 128, 200])
def test_head_norm_rope_sum_order_is_the_reference_shuffle_pattern(D):
    """Inputs whose squares span many binades, so the association order shows in the
    float32 sum: the oracle's rstd must come from the shuffle-pattern sum."""
    S, H = 3, 1
    rng = np.random.default_rng(D)
    xf = (rng.standard_normal((S, D)) * np.exp2(rng.integers(-12, 12, (S, D)))).astype(np.float32)
    x = oracle.f32_to_bf16(xf)
    w = np.ones(D, np.float32)
    out = oracle.bf16_to_f32(oracle.head_norm_rope(x, S, D, 0, H, D, norm_w=w, eps=1e-5))
    xb = oracle.bf16_to_f32(x)
    for s in range(S):
        ss = _shfl_xor_block_sum((xb[s] * xb[s]).astype(np.float32), D)
        rstd = np.float32(1.0 / np.sqrt(np.float64(np.float32(ss / np.float32(D)) + np.float32(1e-5))))
        want = oracle.bf16_to_f32(oracle.f32_to_bf16((xb[s] * rstd).astype(np.float32)))
        assert np.array_equal(out[s, 0], want)


def test_f16_conversion_matches_numpy():
    """or_f32_to_f16 (the split partials' storage) is IEEE round-to-nearest-even: equal
    to numpy's float32 -> float16 cast on hand cases (ties, subnormals, overflow) and
    random values over the whole range; or_f16_to_f32 inverts it exactly."""
    hand = [0.0, -0.0, 1.0, -2.5, 65504.0, 65519.99, 65520.0, 1e9, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -25,
            2.0 ** -14, 2.0 ** -14 - 2.0 ** -26, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 448.0 * (1 + 2.0 ** -4),
            float("inf"), -float("inf")]
    rng = np.random.default_rng(5)
    vals = np.concatenate([np.array(hand, np.float32),
                           (rng.standard_normal(4000) * np.exp2(rng.uniform(-30, 17, 4000))).astype(np.float32)])
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f16(float(x)) for x in vals], np.uint16)
    assert np.array_equal(got, want)
    back = np.array([oracle.f16_to_f32(int(h)) for h in want], np.float32)
    assert np.array_equal(back, want.view(np.float16).astype(np.float32))
    assert oracle.f16(float("nan")) & 0x7C00 == 0x7C00 and oracle.f16(float("nan")) & 0x3FF


def test_sage_split_merge_duplicated_keys():
    """Split merge pinned by an invariant: K/V = [X; X] split into two parts at the
    copy boundary gives each part the (m, l, acc) of X alone, so the merge has
    w = 1, l = 2 l_X and the output equals the unsplit output over X up to the fp16
    storage of the normalised partial (relative 2^-11). A wrong weight, a dropped part
    or l taken from one part only gives an error of order 1."""
    rng = np.random.default_rng(21)
    Sq, n, H, D = 40, 192, 2, 128
    q = _bf16_rand(rng, (Sq, H, D)); k = _bf16_rand(rng, (n, H, D)); v = _bf16_rand(rng, (n, H, D))
    _, t = oracle.sage_reference(q, k, v, Sq, n, H, H, D, rows=np.zeros(0, np.int32))
    ki2 = np.concatenate([t["ki"], t["ki"]], axis=1)
    vt2 = np.concatenate([t["vt"], t["vt"]], axis=2)
    ks2 = np.concatenate([t["ks"], t["ks"]], axis=1)
    args = (t["qi"], t["ki"], t["vt"], t["qs"], t["ks"], t["va"], Sq, n, H, H, D)
    one = oracle.sage_emulate(*args, headroom=oracle.KERNEL_HEADROOM)
    two = oracle.sage_emulate(t["qi"], ki2, vt2, t["qs"], ks2, t["va"], Sq, 2 * n, H, H, D,
                              headroom=oracle.KERNEL_HEADROOM, split=(0, 2))
    assert np.allclose(two, one, rtol=2.0 ** -10, atol=1e-6 * np.abs(one).max())
    assert not np.array_equal(two, one)  # the fp16 storage is really there
    # unsplit over [X; X]: the same softmax up to the running-max path, not bitwise
    seq = oracle.sage_emulate(t["qi"], ki2, vt2, t["qs"], ks2, t["va"], Sq, 2 * n, H, H, D,
                              headroom=oracle.KERNEL_HEADROOM)
    assert cosine(seq, one) > 0.9999


def test_sage_split_merge_one_live_part():
    """A split unit whose other parts see only padded keys (m = -inf, l = 0) merges to
    the output of the part that holds the live keys, computed unsplit over those keys
    (up to the fp16 storage of the partial); with no live key at all the output is 0."""
    rng = np.random.default_rng(22)
    Sq, Skv, H, D = 16, 256, 1, 128
    q = _bf16_rand(rng, (Sq, H, D)); k = _bf16_rand(rng, (Skv, H, D)); v = _bf16_rand(rng, (Skv, H, D))
    mask = np.zeros(Skv, np.uint8); mask[192:] = 1  # only the last of 4 parts is live
    _, t = oracle.sage_reference(q, k, v, Sq, Skv, H, H, D, kv_valid=mask, rows=np.zeros(0, np.int32))
    args = (t["qi"], t["ki"], t["vt"], t["qs"], t["ks"], t["va"], Sq, Skv, H, H, D)
    seq = oracle.sage_emulate(*args, kv_valid=mask, headroom=oracle.KERNEL_HEADROOM)
    split = oracle.sage_emulate(*args, kv_valid=mask, headroom=oracle.KERNEL_HEADROOM, split=(0, 4))
    assert np.allclose(split, seq, rtol=2.0 ** -10, atol=1e-6 * np.abs(seq).max())
    none = oracle.sage_emulate(*args, kv_valid=np.zeros(Skv, np.uint8), split=(0, 4))
    assert np.all(none == 0)


# ---------------- MXFP8 block-scaled quantizer / GEMM (reference src/kernels/blockscale.cu) ----------------

def _e4m3_lut():
    return np.array([oracle.e4m3_to_f32(c) for c in range(256)], np.float64)


def test_mxfp8_quantizer_scale_rule_and_exact_values():
    """Scale = the smallest power of two with bmax / 2^e <= 448 (checked against float64
    log2, independent of the frexp formulation), padding of the rule's edge cases, and
    blocks whose values are e4m3 numbers times 2^k round-trip exactly."""
    rng = np.random.default_rng(31)
    rows, K = 6, 256
    x = (rng.standard_normal((rows, K)) * np.exp2(rng.integers(-20, 20, (rows, 1)))).astype(np.float32)
    x[0, :32] = 0.0                                     # zero block -> e = -127, q = 0
    x[1, :32] = 0.0; x[1, 5] = 448.0 * 2.0 ** 3         # bmax / 448 a power of two -> e = 3, q = 448
    x[1, 32:64] = 0.0; x[1, 40] = -448.0 * 2.0 ** -5 * 1.0078125  # just above -> e = -4
    t = _e4m3_lut()
    x[2, :32] = t[rng.integers(1, 0x7E, 32)] * 2.0 ** 7  # exact e4m3 values x 2^7
    xb = oracle.f32_to_bf16(x)
    q, sf = oracle.mxfp8_quantize(xb, rows, K)
    xf = oracle.bf16_to_f32(xb).astype(np.float64)
    bmax = np.abs(xf.reshape(rows, K // 32, 32)).max(-1)
    with np.errstate(divide="ignore"):
        want = np.where(bmax > 0, np.ceil(np.log2(bmax / 448.0)), -127).clip(-127, 127)
    assert np.array_equal(sf.astype(np.int64) - 127, want.astype(np.int64))
    assert sf[0, 0] == 0 and np.all(q[0, :32] == 0)
    assert sf[1, 0] == 127 + 3 and q[1, 5] == 0x7E
    assert sf[1, 1] == 127 - 4
    deq = t[q].reshape(rows, K // 32, 32) * np.exp2(sf.astype(np.float64) - 127)[..., None]
    np.testing.assert_array_equal(deq.reshape(rows, K)[2, :32], xf[2, :32])
    # nearest-even rounding to the e4m3 grid of the block: error <= half an e4m3 ulp
    err = np.abs(deq.reshape(rows, K) - xf)
    scale = np.exp2(sf.astype(np.float64) - 127).repeat(32, axis=1)
    assert np.all(err <= np.maximum(np.abs(xf) * 2.0 ** -4, scale * 2.0 ** -10) * (1 + 1e-12))


def test_mx_scale_layout():
    """The interleaved scale layout: a bijection onto pad128(rows) x pad4(K/32) bytes, the
    reference quantizer's row base (blockscale.cu:82: sf + (r/128) nkb_pad 128 + (r%32) 16 +
    ((r%128)/32) 4) plus its decoder's block term ((kb/4) 512 + kb%4, blockscale_test.cpp:16)
    at hand-picked points, and pack / unpack inverse to each other."""
    rows, K = 300, 32 * 10                       # nkb = 10 -> padded to 12, rows padded to 384
    nkp = 12
    r, kb = np.meshgrid(np.arange(384), np.arange(nkp), indexing="ij")
    off = oracle.mx_sf_offset(r, kb, nkp).reshape(-1)
    assert np.array_equal(np.sort(off), np.arange(384 * nkp))
    f = lambda a, b: int(oracle.mx_sf_offset(a, b, nkp))
    assert [f(0, 0), f(0, 1), f(0, 3), f(0, 4), f(1, 0), f(31, 0), f(32, 0), f(96, 0), f(127, 3), f(128, 0)] == \
        [0, 1, 3, 512, 16, 496, 4, 12, 511, 128 * nkp]
    assert f(130, 5) == 128 * nkp + 512 + 2 * 16 + 1
    sf = np.random.default_rng(5).integers(0, 255, (rows, K // 32)).astype(np.uint8)
    buf = oracle.mx_scale_pack(sf, rows, K)
    assert buf.size == 384 * nkp and np.array_equal(oracle.mx_scale_unpack(buf, rows, K), sf)
    assert np.count_nonzero(buf == 127) >= 384 * nkp - rows * (K // 32)


def test_mxfp8_gemm_oracle_matches_numpy():
    """The GEMM oracle against a numpy float64 restatement (dequantize, matmul), and the
    identity: W = I with unit scales returns the dequantized X."""
    rng = np.random.default_rng(32)
    M, N, K = 7, 5, 96
    xb = oracle.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32) * 3)
    wb = oracle.f32_to_bf16(rng.standard_normal((N, K)).astype(np.float32) * 0.1)
    xq, xs = oracle.mxfp8_quantize(xb, M, K)
    wq, ws = oracle.mxfp8_quantize(wb, N, K)
    t = _e4m3_lut()
    dq = lambda q, s: (t[q].reshape(q.shape[0], -1, 32) * np.exp2(s.astype(np.float64) - 127)[..., None]).reshape(q.shape)
    want = dq(xq, xs) @ dq(wq, ws).T
    got = oracle.gemm_mxfp8(wq, ws, xq, xs, M, N, K)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-9)
    eye = np.zeros((K, K), np.uint8); eye[np.arange(K), np.arange(K)] = 0x38  # e4m3 1.0
    ones = np.full((K, K // 32), 127, np.uint8)
    got = oracle.gemm_mxfp8(eye, ones, xq, xs, M, K, K)
    np.testing.assert_array_equal(got, dq(xq, xs).astype(np.float32))


# ---------------- NVFP4 (reference src/kernels/blockscale.cu, NVFP4 branch) ----------------

_E2M1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float64)


def _e2m1_decode(codes):
    """The reference test's decoder (tests/blockscale_test.cpp:37-43): sign bit 8,
    magnitude table {0, 0.5, 1, 1.5, 2, 3, 4, 6}."""
    codes = np.asarray(codes)
    return np.where(codes & 8, -1.0, 1.0) * _E2M1[codes & 7]


def test_e2m1_is_nearest_even_by_search():
    """Every midpoint and random values: the code of the nearest e2m1 magnitude, ties to
    the even code, saturating at 6; the sign bit for negative values."""
    mids = (_E2M1[:-1] + _E2M1[1:]) / 2
    rng = np.random.default_rng(41)
    xs = np.concatenate([mids, -mids, _E2M1, -_E2M1[1:], rng.uniform(-8, 8, 2000), [6.5, 100.0, -1e9]])
    for x in xs.astype(np.float32):
        a = abs(float(x))
        d = np.abs(_E2M1 - min(a, 6.0))
        best = np.flatnonzero(d == d.min())
        code = int(best[0]) if len(best) == 1 else int([b for b in best if b % 2 == 0][0])
        want = code | (8 if x < 0 else 0)
        assert oracle.e2m1(x) == want, (x, oracle.e2m1(x), want)
        assert oracle.e2m1_to_f32(want) == _e2m1_decode(want)


def test_nvfp4_quantizer_rules():
    """amax = max |x| (numpy); the tensor's largest element gets scale 448 and code 6; a
    zero block gets scale 0 and codes 0; every block scale is the e4m3 of float64
    bmax / (6 g) up to the float rounding of the reference's single-precision steps (one
    e4m3 step at most, only where float64 lands within 1e-6 of a rounding boundary);
    elements decode to within half an e2m1 step of x / sd, or saturate at 6."""
    rng = np.random.default_rng(42)
    rows, K = 5, 160
    x = (rng.standard_normal((rows, K)) * np.exp2(rng.integers(-6, 6, (rows, 1)))).astype(np.float32)
    x[0, :16] = 0.0
    x[3, 37] = 1000.0
    xb = oracle.f32_to_bf16(x)
    q, sf, amax = oracle.nvfp4_quantize(xb, rows, K)
    xf = oracle.bf16_to_f32(xb).astype(np.float64)
    assert amax == np.abs(xf).max() == 1000.0
    g = amax / (6 * 448)
    codes = np.stack([q & 15, q >> 4], -1).reshape(rows, K)
    t = _e4m3_lut()
    assert sf[3, 37 // 16] == 0x7E and codes[3, 37] == 7        # 448 and +6
    assert sf[0, 0] == 0 and np.all(codes[0, :16] == 0)
    bmax = np.abs(xf.reshape(rows, K // 16, 16)).max(-1)
    near = np.array([[oracle.e4m3(np.float32(b / (6 * g))) for b in row] for row in bmax])
    assert np.all(np.abs(sf.astype(np.int64) - near.astype(np.int64)) <= 1)
    sd = t[sf] * g
    y = xf.reshape(rows, K // 16, 16) / np.where(sd > 0, sd, 1)[..., None]
    dec = _e2m1_decode(codes).reshape(rows, K // 16, 16)
    step = np.where(np.abs(y) < 2, 0.5, np.where(np.abs(y) < 4, 1.0, 2.0))
    ok = (np.abs(dec - y) <= step / 2 * (1 + 1e-6)) | ((np.abs(dec) == 6) & (np.abs(y) >= 5))
    assert np.all(ok | (sd[..., None] == 0))
    # amax = 0: g = 1, every scale and code 0
    q0, sf0, a0 = oracle.nvfp4_quantize(np.zeros((2, 32), np.uint16), 2, 32)
    assert a0 == 0.0 and not q0.any() and not sf0.any()


def test_nvfp4_gemm_oracle_matches_numpy():
    """The GEMM oracle against a numpy float64 decode (the reference test's decoder) and
    matmul, scaled by alpha = gW gX."""
    rng = np.random.default_rng(43)
    M, N, K = 6, 5, 96
    xb = oracle.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32) * 3)
    wb = oracle.f32_to_bf16(rng.standard_normal((N, K)).astype(np.float32) * 0.02)
    xq, xs, xa = oracle.nvfp4_quantize(xb, M, K)
    wq, ws, wa = oracle.nvfp4_quantize(wb, N, K)
    t = _e4m3_lut()

    def dq(q, s, amax):
        codes = np.stack([q & 15, q >> 4], -1).reshape(q.shape[0], -1)
        g = np.float32(amax) / np.float32(6 * 448)
        return (_e2m1_decode(codes).reshape(q.shape[0], -1, 16) * t[s][..., None]).reshape(codes.shape), g

    dx, gx = dq(xq, xs, xa)
    dw, gw = dq(wq, ws, wa)
    want = (dx @ dw.T) * float(np.float32(gx * gw))
    got = oracle.gemm_nvfp4(wq, ws, wa, xq, xs, xa, M, N, K)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-12)
    # and the decoded product approximates the bf16 GEMM (the reference's gate: 15 %)
    ref = oracle.bf16_to_f32(xb).astype(np.float64) @ oracle.bf16_to_f32(wb).astype(np.float64).T
    assert np.sqrt(((got - ref) ** 2).sum() / (ref ** 2).sum()) < 0.15

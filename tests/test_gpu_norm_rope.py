"""GPU parity of head_norm_rope (mx_head_norm_rope through the C ABI) against the
oracle's restatement of the reference kernel (src/kernels/ops.cu:87-119)."""
import numpy as np
import pytest
import torch

import oracle
from miroxen_amd import ROPE_HALF, ROPE_INTERLEAVED, ROPE_NONE, head_norm_rope

pytestmark = pytest.mark.gpu

# S, H, D, rot, mode, norm, col0, stride_extra
CASES = [
    (300, 24, 128, 128, ROPE_INTERLEAVED, True, 0, 0),     # Qwen-Image q/k
    (257, 8, 128, 128, ROPE_HALF, True, 128, 384),         # Qwen3 text (k slice of a fused row)
    (500, 16, 72, 72, ROPE_HALF, False, 0, 72 * 32),        # Qwen3-VL vision (no norm)
    (99, 40, 128, 64, ROPE_HALF, True, 0, 0),               # partial rotary (H3 style)
    (33, 4, 64, 0, ROPE_NONE, True, 8, 8),                  # norm only
    (17, 2, 256, 256, ROPE_INTERLEAVED, True, 0, 0),        # largest D
    (65, 3, 100, 40, ROPE_INTERLEAVED, True, 0, 0),         # D not a multiple of 32
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"S{c[0]}H{c[1]}D{c[2]}r{c[3]}m{c[4]}{'n' if c[5] else ''}")
def test_head_norm_rope_matches_oracle(cuda, case):
    S, H, D, rot, mode, norm, col0, extra = case
    print(f"head_norm_rope case {case}", flush=True)
    rng = np.random.default_rng(S * 7 + D)
    stride = col0 + H * D + extra
    x = oracle.f32_to_bf16((rng.standard_normal((S, stride)) * 1.5).astype(np.float32))
    w = rng.uniform(0.5, 1.5, D).astype(np.float32) if norm else None
    cs = sn = None
    if rot:
        ang = rng.uniform(-np.pi, np.pi, (S, rot // 2))
        cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    want = oracle.head_norm_rope(x, S, stride, col0, H, D, norm_w=w, eps=1e-6, cos=cs, sin=sn, rot=rot, mode=mode)
    dev = lambda a: None if a is None else torch.from_numpy(a).to(cuda)
    xin = torch.from_numpy(x.view(np.int16)).to(cuda)
    out = torch.full((S * H * D + 64,), -1, dtype=torch.int16, device=cuda)
    head_norm_rope(xin, S, stride, col0, H, D, dev(w), 1e-6, dev(cs), dev(sn), rot, mode, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.all(got[S * H * D:] == -1), "wrote past the output"
    got = got[: S * H * D].view(np.uint16).reshape(S, H, D)
    gf, wf = oracle.bf16_to_f32(got).astype(np.float64), oracle.bf16_to_f32(want).astype(np.float64)
    # The reference's rsqrtf and this build's v_rsq_f32 both approximate the correctly
    # rounded rsqrt the oracle uses, and the rotation's a*c - b*s may be contracted to
    # an FMA: results are one bf16 rounding step apart, plus fp32-level differences
    # that show only where the rotation cancels (tolerance relative to the row scale).
    row = np.max(np.abs(wf), axis=-1, keepdims=True)
    assert np.all(np.abs(gf - wf) <= np.abs(wf) * 2.0 ** -7 + row * 2.0 ** -14)
    assert np.mean(got == want) >= 0.98


def test_head_norm_rope_empty_is_noop(cuda):
    out = torch.full((8,), 7, dtype=torch.int16, device=cuda)
    head_norm_rope(out, 0, 128, 0, 1, 128, None, 0.0, None, None, 0, ROPE_NONE, out)
    torch.cuda.synchronize()
    assert torch.all(out == 7)


# ---- fused head_norm_rope + Sage prologue (mx_sage_quantize_norm_rope) ----
# S, H, rot, mode, q_norm, k_norm, masked
FUSED = [
    (300, 4, 128, ROPE_INTERLEAVED, True, True, False),   # Qwen-Image q/k
    (1000, 3, 64, ROPE_HALF, True, True, True),           # H3-style partial rotate-half, key mask
    (257, 2, 0, ROPE_NONE, True, False, False),           # norm only (Q)
    (130, 2, 32, ROPE_INTERLEAVED, False, True, False),   # partial interleaved rope, K norm only
    (4352, 2, 128, ROPE_HALF, True, True, False),         # config-2 length, full rotate-half
]


@pytest.mark.parametrize("case", FUSED, ids=lambda c: f"S{c[0]}H{c[1]}r{c[2]}m{c[3]}")
def test_fused_norm_rope_prologue_is_bit_exact(cuda, case):
    """Fused prologue == head_norm_rope(q), head_norm_rope(k), then the plain Sage prologue
    and kernel: every workspace region and the attention output bit for bit. q, k, v are
    slices of one fused QKV projection row [S, 3HD], as in the reference's DiT blocks
    (src/models/minimax_h3/dit.cpp:210-212)."""
    from miroxen_amd import (AttnParams, flash_attn_fp8, flash_attn_fp8_norm_rope, flash_attn_fp8_workspace,
                             sage_layout, sage_quantize, sage_quantize_norm_rope)
    S, H, rot, mode, qn, kn, masked = case
    D = 128
    print(f"fused norm/rope prologue {case}", flush=True)
    rng = np.random.default_rng(S + rot)
    HD = H * D
    t = oracle.f32_to_bf16((rng.standard_normal((S, 3 * HD)) * 1.5).astype(np.float32))
    tt = torch.from_numpy(t.view(np.int16)).view(torch.bfloat16).to(cuda)
    qw = torch.from_numpy(rng.uniform(0.5, 1.5, D).astype(np.float32)).to(cuda) if qn else None
    kw = torch.from_numpy(rng.uniform(0.5, 1.5, D).astype(np.float32)).to(cuda) if kn else None
    cs = sn = None
    if rot:
        ang = rng.uniform(-np.pi, np.pi, (S, rot // 2))
        cs = torch.from_numpy(np.cos(ang).astype(np.float32)).to(cuda)
        sn = torch.from_numpy(np.sin(ang).astype(np.float32)).to(cuda)
    mask = None
    if masked:
        mask = torch.from_numpy((rng.random(S) > 0.15).astype(np.uint8)).to(cuda)
    eps = 1e-6
    # two-step reference path on this device
    qd = torch.empty(S, HD, dtype=torch.bfloat16, device=cuda)
    kd = torch.empty_like(qd)
    head_norm_rope(tt, S, 3 * HD, 0, H, D, qw, eps, cs, sn, rot, mode, qd)
    head_norm_rope(tt, S, 3 * HD, HD, H, D, kw, eps, cs, sn, rot, mode, kd)
    vd = tt[:, 2 * HD:].contiguous()
    p2 = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=D, kv_valid=mask)
    n = flash_attn_fp8_workspace(p2)
    ws2 = torch.zeros(n, dtype=torch.uint8, device=cuda)
    sage_quantize(qd, kd, vd, p2, ws2)
    o2 = torch.empty_like(qd)
    flash_attn_fp8(qd, kd, vd, o2, p2, ws2)
    # fused path on the raw projections
    p1 = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=D, q_stride=3 * HD, kv_stride=3 * HD, o_stride=HD, kv_valid=mask)
    ws1 = torch.zeros(flash_attn_fp8_workspace(p1), dtype=torch.uint8, device=cuda)
    base = tt.data_ptr()
    qp, kp, vp = base, base + 2 * HD, base + 4 * HD  # bytes: bf16 columns 0, HD, 2HD
    sage_quantize_norm_rope(qp, kp, vp, p1, qw, kw, eps, cs, sn, rot, mode, ws1)
    o1 = torch.empty_like(qd)
    flash_attn_fp8_norm_rope(qp, kp, vp, o1, p1, qw, kw, eps, cs, sn, rot, mode, ws1)
    torch.cuda.synchronize()
    L1, L2 = sage_layout(p1), sage_layout(p2)
    for name, cnt, dt in (("qi", H * L1["sq_pad"] * D, np.int8), ("ki", H * L1["skv_pad"] * D, np.int8),
                          ("vt", H * D * L1["skv_pad"], np.uint8), ("qs", H * L1["sq_pad"] // 16, np.float32),
                          ("ks", H * L1["skv_pad"] // 64, np.float32), ("km", H * D, np.float32),
                          ("va", H * D, np.float32)):
        nb = cnt * np.dtype(dt).itemsize
        a = ws1[L1[name]: L1[name] + nb].cpu().numpy()
        b = ws2[L2[name]: L2[name] + nb].cpu().numpy()
        assert np.array_equal(a, b), name
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))

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

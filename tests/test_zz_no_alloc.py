"""mx_flash_attn_fp8_noalloc through the C ABI: the quantized attention with the
workspace in the library's fixed device scratch instead of a caller allocation. Its
output must equal mx_flash_attn_fp8's with a caller workspace bit for bit (same
prologue, same kernels, same workspace layout), on two calls in a row, the second
with a smaller input, and a shape whose workspace exceeds the scratch is refused."""
import ctypes

import pytest
import torch

from miroxen_amd import _lib
from miroxen_amd.attention import AttnParams, flash_attn_fp8_workspace
from miroxen_amd.synth import CONFIGS, make_inputs

pytestmark = pytest.mark.gpu


def _call_ref(q, k, v, o, p, ws):
    c = p.c()
    rc = _lib.load().mx_flash_attn_fp8(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), ctypes.byref(c),
                                       ws.data_ptr(), None)
    assert rc == 0, _lib.load().mx_last_error()


def _call_noalloc(q, k, v, o, p):
    c = p.c()
    return _lib.load().mx_flash_attn_fp8_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                                 ctypes.byref(c), None)


def _case(cfg, seed, dev):
    q, k, v, mask = make_inputs(cfg, seed=seed, device=dev)
    p = AttnParams(Sq=cfg.S, Skv=cfg.S, Hq=cfg.H, Hkv=cfg.H, D=cfg.D, kv_valid=mask)
    return q, k, v, p


def test_noalloc_matches_workspace_entry(cuda):
    # config 3 (masked, split grid), then config 1 (smaller: the scratch keeps the
    # larger call's bytes past the smaller layout)
    for cfg_id in (3, 1):
        cfg = CONFIGS[cfg_id]
        print(f"noalloc config {cfg_id} {cfg.name}", flush=True)
        q, k, v, p = _case(cfg, cfg_id, cuda)
        ws = torch.empty(flash_attn_fp8_workspace(p), dtype=torch.uint8, device=cuda)
        want = torch.empty_like(q)
        _call_ref(q, k, v, want, p, ws)
        got = torch.full_like(q, float("nan"))
        rc = _call_noalloc(q, k, v, got, p)
        assert rc == 0, _lib.load().mx_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"config {cfg_id}"


def test_noalloc_refuses_oversize_workspace(cuda):
    S, H, D = 16384, 24, 128  # workspace of about 146 MiB
    p = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=D)
    assert flash_attn_fp8_workspace(p) > 128 << 20
    q = torch.zeros(S, H * D, dtype=torch.bfloat16, device=cuda)
    rc = _call_noalloc(q, q, q, q, p)
    assert rc == _lib.MX_E_UNSUPPORTED
    assert b"exceeds" in _lib.load().mx_last_error()

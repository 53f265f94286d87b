"""mx_flash_attn_fp8_noalloc through the C ABI: the quantized attention with the
workspace in the library's fixed device scratch instead of a caller allocation. Its
output must equal mx_flash_attn_fp8's with a caller workspace bit for bit (same
prologue, same kernels, same workspace layout), on two calls in a row, the second
with a smaller input, and a shape whose workspace exceeds the scratch is refused.
Calls on two streams are ordered by the library's event; the fallback to
mx_flash_attn (arguments the quantized path does not take) allocates nothing either."""
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


def test_noalloc_calls_on_two_streams(cuda):
    """Two shapes on two streams, back to back without host sync between them: the
    second call waits (on the device) for the first, so neither overwrites the other's
    workspace and both equal their workspace-entry results bit for bit."""
    cases = []
    for cfg_id in (1, 3):
        cfg = CONFIGS[cfg_id]
        q, k, v, p = _case(cfg, 40 + cfg_id, cuda)
        ws = torch.empty(flash_attn_fp8_workspace(p), dtype=torch.uint8, device=cuda)
        want = torch.empty_like(q)
        _call_ref(q, k, v, want, p, ws)
        cases.append((q, k, v, p, want, torch.empty_like(q)))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for it in range(3):
        print(f"noalloc two streams, iteration {it}", flush=True)
        for (q, k, v, p, _, got), st in zip(cases, streams):
            got.fill_(float("nan"))
            st.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(st):
                c = p.c()
                rc = _lib.load().mx_flash_attn_fp8_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), got.data_ptr(),
                                                           ctypes.byref(c), ctypes.c_void_p(st.cuda_stream))
                assert rc == 0, _lib.load().mx_last_error()
        torch.cuda.synchronize()
        for q, k, v, p, want, got in cases:
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (it, p.Sq)


def test_noalloc_fallback_allocates_nothing(cuda):
    """D = 72 is not a quantized-path shape: the call falls back to mx_flash_attn, here
    on a grid of few units that runs split. The free device memory does not change and
    the output equals mx_flash_attn's bit for bit."""
    from miroxen_amd.attention import flash_attn, flash_attn_split_plan
    Sq, Skv, H, D = 512, 4096, 4, 72
    g = torch.Generator(device=cuda); g.manual_seed(77)
    q, k, v = (torch.randn(S_, H * D, generator=g, device=cuda).to(torch.bfloat16) for S_ in (Sq, Skv, Skv))
    p = AttnParams(Sq=Sq, Skv=Skv, Hq=H, Hkv=H, D=D)
    assert flash_attn_split_plan(p)[2] > 1
    want, got = torch.empty_like(q), torch.full_like(q, float("nan"))
    flash_attn(q, k, v, want, p)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    assert _call_noalloc(q, k, v, got, p) == 0, _lib.load().mx_last_error()
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))

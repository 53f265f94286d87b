"""GPU parity of the one-pass K/V prologue (prep_kv_fused): eager calls run it, calls
under stream capture run the three-launch prologue (statistics blocks, finalization,
K/V quantizer). Both must fill the workspace bit for bit alike, and both must equal
the oracle's restatement of the reference quantizer (src/kernels/attention_fp8.cu:51-127):
 * up to 32 blocks of 256 keys per head (the one-pass path) and beyond (the
   three-launch path runs eagerly too);
 * ragged key counts, padded strides, GQA, masks, D = 64 and 128;
 * a workspace full of stale bytes (ready flags are per-call epochs, never cleared),
   and repeated calls on one workspace."""
import numpy as np
import pytest
import torch

import oracle
from miroxen_amd import AttnParams, flash_attn_fp8, sage_layout, sage_quantize
from tests.test_gpu_sage import _bias_inputs, _bits, _quantized, _ws

pytestmark = pytest.mark.gpu

REGIONS = ("km", "va", "qs", "ks", "qi", "ki", "vt")


def _tab(ws, p, L):
    """Tile-table entries of the key tiles (each head's row has one spare slot after them
    that no prologue writes)."""
    nt = L["skv_pad"] // 64
    n = p.Hkv * (nt + 1) * 16
    return ws[L["tab"]: L["tab"] + n].cpu().numpy().reshape(p.Hkv, nt + 1, 16)[:, :nt]


def _captured_quantize(q, k, v, p, ws, replays=3):
    """sage_quantize captured in a graph (the three-launch prologue), replayed with eager
    fused-prologue work on another workspace between replays; returns every replay's
    workspace copy."""
    other = torch.zeros_like(ws)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        sage_quantize(q, k, v, p, ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        sage_quantize(q, k, v, p, ws)
    outs = []
    for _ in range(replays):
        ws.fill_(0xA5)
        g.replay()
        torch.cuda.synchronize()
        outs.append(ws.clone())
        sage_quantize(q, k, v, p, other)  # eager work between replays
        torch.cuda.synchronize()
    return outs


# Sq, Skv, Hq, Hkv, D, pad, kbias, masked: blocks of 256 keys per head = ceil(Skv / 256)
CASES = [
    (64, 1, 2, 2, 128, 0, 0.0, False),        # one key
    (130, 1000, 4, 2, 128, 5, 4.0, True),     # 4 blocks, GQA, padded stride, mask
    (77, 8192, 2, 2, 128, 0, 2.0, False),     # 32 blocks: the last fold-mode size
    (77, 8193, 2, 2, 128, 8, 2.0, True),      # 33 blocks: three-launch path
    (33, 12544, 3, 3, 128, 0, 8.0, True),     # config 4's key count (49 blocks)
    (300, 777, 4, 4, 64, 0, 4.0, True),       # D = 64
    (40, 8000, 2, 2, 64, 3, 2.0, False),      # D = 64, 32 blocks
]


def _case_id(c):
    return f"{c[0]}x{c[1]}_h{c[2]}-{c[3]}_d{c[4]}_p{c[5]}{'_m' if c[7] else ''}"


@pytest.mark.parametrize("case", CASES, ids=_case_id)
def test_fused_prologue_bit_exact(cuda, case):
    Sq, Skv, Hq, Hkv, D, pad, kbias, masked = case
    print(f"fused prologue {_case_id(case)}", flush=True)
    q, k, v, qs, ks = _bias_inputs(Sq, Skv, Hq, Hkv, D, pad, kbias, cuda, Skv * 7 + Hq)
    mask = None
    if masked:
        mask = (torch.rand(Skv, generator=torch.Generator().manual_seed(Skv + 1)) > 0.2).to(torch.uint8).to(cuda)
    p = AttnParams(Sq=Sq, Skv=Skv, Hq=Hq, Hkv=Hkv, D=D, q_stride=qs, kv_stride=ks, o_stride=qs, kv_valid=mask)
    L = sage_layout(p)
    ws = _ws(p, cuda)
    ws.fill_(0xFF)  # stale bytes everywhere, flags included
    sage_quantize(q, k, v, p, ws)
    torch.cuda.synchronize()
    eager = _quantized(ws, p, L)
    tab = _tab(ws, p, L)
    # the oracle's restatement of the reference quantizer
    _, want = oracle.sage_reference(_bits(q), _bits(k), _bits(v), Sq, Skv, Hq, Hkv, D, q_stride=qs, kv_stride=ks,
                                    rows=np.zeros(0, np.int32))
    for name in REGIONS:
        assert np.array_equal(eager[name], want[name]), f"{name} differs from the reference quantizer"
    # a second call on the same workspace (old flags of the first call in place)
    sage_quantize(q, k, v, p, ws)
    torch.cuda.synchronize()
    again = _quantized(ws, p, L)
    for name in REGIONS:
        assert np.array_equal(again[name], eager[name]), f"{name}: second call differs"
    assert np.array_equal(_tab(ws, p, L), tab)
    # the captured (three-launch) prologue: every replay equals the eager workspace
    for i, w in enumerate(_captured_quantize(q, k, v, p, torch.empty_like(ws))):
        got = _quantized(w, p, L)
        for name in REGIONS:
            assert np.array_equal(got[name], eager[name]), f"replay {i}: {name} differs from the eager prologue"
        assert np.array_equal(_tab(w, p, L), tab), f"replay {i}: tile table differs"


def test_fused_prologue_random_stale_workspace(cuda):
    """A workspace of random bytes (as a fresh caller allocation may hold) and the
    attention output of flash_attn_fp8 on it: equal to the output on a zeroed one."""
    Sq = Skv = 4352
    H = 4
    q, k, v, qs, ks = _bias_inputs(Sq, Skv, H, H, 128, 0, 4.0, cuda, 99)
    p = AttnParams(Sq=Sq, Skv=Skv, Hq=H, Hkv=H, D=128)
    ws1, ws2 = _ws(p, cuda), _ws(p, cuda)
    ws2.copy_(torch.randint(0, 256, ws2.shape, dtype=torch.uint8, generator=torch.Generator().manual_seed(5))
              .to(cuda))
    o1 = torch.empty((Sq, H * 128), dtype=torch.bfloat16, device=cuda)
    o2 = torch.empty_like(o1)
    flash_attn_fp8(q, k, v, o1, p, ws1)
    flash_attn_fp8(q, k, v, o2, p, ws2)
    torch.cuda.synchronize()
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))


def test_fused_prologue_recompute_path(cuda):
    """The bounded wait forced to one look (test hook): work-groups that do not yet see
    every flag of their head compute the missing partials from K and V themselves. The
    workspace is the same bit for bit (config-3 shape, 17 blocks per head)."""
    from miroxen_amd import _lib
    Sq = Skv = 4352
    H = 8
    q, k, v, qs, ks = _bias_inputs(Sq, Skv, H, H, 128, 0, 8.0, cuda, 7)
    p = AttnParams(Sq=Sq, Skv=Skv, Hq=H, Hkv=H, D=128)
    L = sage_layout(p)
    ws1, ws2 = _ws(p, cuda), _ws(p, cuda)
    sage_quantize(q, k, v, p, ws1)
    lib = _lib.load()
    _lib.check(lib.mx_sage_prologue_wait_ticks(0))
    try:
        for _ in range(3):
            ws2.fill_(0)
            sage_quantize(q, k, v, p, ws2)
            torch.cuda.synchronize()
            a, b = _quantized(ws1, p, L), _quantized(ws2, p, L)
            for name in REGIONS:
                assert np.array_equal(a[name], b[name]), name
            assert np.array_equal(_tab(ws1, p, L), _tab(ws2, p, L))
    finally:
        _lib.check(lib.mx_sage_prologue_wait_ticks(20000))


def _random_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        Skv = int(rng.integers(1, 8193))
        Hkv = int(rng.choice([1, 2, 3, 4]))
        Hq = Hkv * int(rng.choice([1, 2]))
        D = int(rng.choice([64, 128]))
        out.append((int(rng.integers(1, 600)), Skv, Hq, Hkv, D, int(rng.choice([0, 3, 8])),
                    float(rng.choice([0.0, 2.0, 8.0])), bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("case", _random_cases(8, 2026), ids=_case_id)
def test_fused_prologue_random_shapes(cuda, case):
    """Seeded random shapes on the one-pass path (Skv <= 8192): every workspace region
    equals the oracle's restatement of the reference quantizer."""
    Sq, Skv, Hq, Hkv, D, pad, kbias, masked = case
    print(f"random fused prologue {_case_id(case)}", flush=True)
    q, k, v, qs, ks = _bias_inputs(Sq, Skv, Hq, Hkv, D, pad, kbias, cuda, Skv + 13 * Sq)
    mask = None
    if masked:
        mask = (torch.rand(Skv, generator=torch.Generator().manual_seed(Skv)) > 0.3).to(torch.uint8).to(cuda)
    p = AttnParams(Sq=Sq, Skv=Skv, Hq=Hq, Hkv=Hkv, D=D, q_stride=qs, kv_stride=ks, o_stride=qs, kv_valid=mask)
    L = sage_layout(p)
    ws = _ws(p, cuda)
    ws.fill_(0x5A)
    sage_quantize(q, k, v, p, ws)
    torch.cuda.synchronize()
    got = _quantized(ws, p, L)
    _, want = oracle.sage_reference(_bits(q), _bits(k), _bits(v), Sq, Skv, Hq, Hkv, D, q_stride=qs, kv_stride=ks,
                                    rows=np.zeros(0, np.int32))
    for name in REGIONS:
        assert np.array_equal(got[name], want[name]), f"{name} differs from the reference quantizer"

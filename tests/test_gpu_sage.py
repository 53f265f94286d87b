"""GPU parity of the Sage INT8/FP8 path (mx_sage_quantize / mx_sage_attend /
mx_flash_attn_fp8 through the C ABI):
 * the quantize prologue bit-exact against the oracle's restatement of the
   reference quantizer (src/kernels/attention_fp8.cu:51-127);
 * the attention kernel against the oracle's emulator of the reference
   arithmetic (:286-416) fed the same workspace, and against exact FP32
   attention (BASELINE: cosine >= 0.995; reference gate rel-RMS < 4 %,
   tests/attention_fp8_test.cpp:65);
 * the reference's fallback contract (:488-500)."""
import numpy as np
import pytest
import torch

import oracle
from miroxen_amd import (AttnParams, flash_attn, flash_attn_fp8, flash_attn_fp8_ok, flash_attn_fp8_supported,
                         flash_attn_fp8_workspace, sage_attend, sage_layout, sage_quantize)
from miroxen_amd.synth import CONFIGS, make_inputs
from tests.helpers import cosine, max_abs, query_rows, rel_rms

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _f32(t):
    return t.float().cpu().numpy()


def _ws(p, dev):
    n = flash_attn_fp8_workspace(p)
    return torch.zeros(n + 256, dtype=torch.uint8, device=dev)[:n] if n else None


def _region(ws, L, name, count, dtype):
    off = L[name]
    return ws[off: off + count * np.dtype(dtype).itemsize].cpu().numpy().view(dtype)


def _quantized(ws, p, L):
    """Read the workspace regions back to host arrays."""
    H, Hk, D = p.Hq, p.Hkv, p.D
    sq, skv = L["sq_pad"], L["skv_pad"]
    return dict(
        qi=_region(ws, L, "qi", H * sq * D, np.int8).reshape(H, sq, D),
        ki=_region(ws, L, "ki", Hk * skv * D, np.int8).reshape(Hk, skv, D),
        vt=_region(ws, L, "vt", Hk * D * skv, np.uint8).reshape(Hk, D, skv),
        qs=_region(ws, L, "qs", H * sq // 16, np.float32).reshape(H, sq // 16),
        ks=_region(ws, L, "ks", Hk * skv // 64, np.float32).reshape(Hk, skv // 64),
        km=_region(ws, L, "km", Hk * D, np.float32).reshape(Hk, D),
        va=_region(ws, L, "va", Hk * D, np.float32).reshape(Hk, D),
    )


def _bias_inputs(Sq, Skv, Hq, Hkv, D, pad, kbias, dev, seed):
    """The reference Sage test generator (tests/attention_fp8_test.cpp:18-27, :49-50):
    N(0,1) plus a per-channel bias (kbias for K, 0.5 for V), strides padded by `pad`."""
    rng = np.random.default_rng(seed)
    qs, ks = Hq * D + pad, Hkv * D + pad
    q = oracle.f32_to_bf16(rng.standard_normal((Sq, qs)).astype(np.float32))
    kb = (rng.standard_normal(ks) * kbias).astype(np.float32)
    k = oracle.f32_to_bf16((rng.standard_normal((Skv, ks)) + kb).astype(np.float32))
    vb = (rng.standard_normal(ks) * 0.5).astype(np.float32)
    v = oracle.f32_to_bf16((rng.standard_normal((Skv, ks)) + vb).astype(np.float32))
    to = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(dev)
    return to(q), to(k), to(v), qs, ks


def test_supported(cuda):
    assert flash_attn_fp8_supported(0)


@pytest.mark.parametrize("Sq,Skv,Hq,Hkv,D,pad,kbias", [
    (1, 1, 1, 1, 128, 0, 0.0), (300, 300, 4, 4, 128, 0, 0.0), (257, 1000, 4, 2, 128, 0, 4.0),
    (130, 77, 2, 2, 128, 8, 2.0), (1088, 1088, 24, 24, 128, 0, 8.0),
    (1, 1, 1, 1, 64, 0, 0.0), (300, 300, 4, 4, 64, 0, 0.0), (257, 1000, 4, 2, 64, 0, 4.0),
    (130, 77, 2, 2, 64, 8, 2.0), (1088, 1088, 24, 24, 64, 0, 8.0),
    (130, 77, 2, 2, 128, 5, 2.0), (257, 300, 4, 2, 64, 5, 4.0),  # strides not multiples of 8
])
def test_prologue_bit_exact(cuda, Sq, Skv, Hq, Hkv, D, pad, kbias):
    print(f"prologue {Sq}x{Skv} H={Hq}/{Hkv} D={D} pad={pad}", flush=True)
    q, k, v, qs, ks = _bias_inputs(Sq, Skv, Hq, Hkv, D, pad, kbias, cuda, Sq * 31 + Skv)
    p = AttnParams(Sq=Sq, Skv=Skv, Hq=Hq, Hkv=Hkv, D=D, q_stride=qs, kv_stride=ks, o_stride=qs)
    ws = _ws(p, cuda)
    sage_quantize(q, k, v, p, ws)
    torch.cuda.synchronize()
    L = sage_layout(p)
    g = _quantized(ws, p, L)
    _, want = oracle.sage_reference(_bits(q), _bits(k), _bits(v), Sq, Skv, Hq, Hkv, D, q_stride=qs, kv_stride=ks,
                                    rows=np.zeros(0, np.int32))
    for name in ("km", "va", "qs", "ks", "qi", "ki", "vt"):
        assert np.array_equal(g[name], want[name]), f"{name} differs from the reference quantizer"


def test_prologue_bit_exact_config3(cuda):
    """Config 3 (outlier K channels, mask) at full size: every quantized byte and scale."""
    cfg = CONFIGS[3]
    q, k, v, mask = make_inputs(cfg, seed=3, device=cuda)
    S, H = cfg.S, cfg.H
    p = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=128, kv_valid=mask)
    ws = _ws(p, cuda)
    sage_quantize(q, k, v, p, ws)
    torch.cuda.synchronize()
    g = _quantized(ws, p, sage_layout(p))
    _, want = oracle.sage_reference(_bits(q), _bits(k), _bits(v), S, S, H, H, 128, rows=np.zeros(0, np.int32))
    for name in ("km", "va", "qs", "ks", "qi", "ki", "vt"):
        assert np.array_equal(g[name], want[name]), name


def test_q_group_64_config3(cuda):
    """Config 3 as its workload states it: one Q scale per 64-token block (q_group=64).
    Every quantized byte and scale against the oracle quantizer with G=64 (the 64-token
    scale sits in each of its four 16-token entries), then the attention against the
    emulator fed that workspace and against exact attention (cosine >= 0.995)."""
    cfg = CONFIGS[3]
    q, k, v, mask = make_inputs(cfg, seed=3, device=cuda)
    S, H = cfg.S, cfg.H
    p = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=128, kv_valid=mask)
    ws = _ws(p, cuda)
    sage_quantize(q, k, v, p, ws, q_group=64)
    torch.cuda.synchronize()
    L = sage_layout(p)
    g = _quantized(ws, p, L)
    _, want = oracle.sage_reference(_bits(q), _bits(k), _bits(v), S, S, H, H, 128, q_group=64,
                                    rows=np.zeros(0, np.int32))
    want["qs"] = np.repeat(want["qs"], 4, axis=1)
    for name in ("km", "va", "qs", "ks", "qi", "ki", "vt"):
        assert np.array_equal(g[name], want[name]), name
    assert np.all(g["qs"][:, 0::4] == g["qs"][:, 3::4])
    o = torch.empty_like(q)
    sage_attend(o, p, ws)
    torch.cuda.synchronize()
    rows = np.array(sorted(set(query_rows(S, H)) | set(range(0, S, S // 40))), np.int32)
    mk = mask.cpu().numpy()
    units = (S + L["split_qt"] - 1) // L["split_qt"] * H
    emu = oracle.sage_emulate(g["qi"], g["ki"], g["vt"], g["qs"], g["ks"], g["va"], S, S, H, H, 128, kv_valid=mk,
                              rows=rows, headroom=oracle.KERNEL_HEADROOM,
                              split=(units - L["split_units"], L["split_parts"], L["split_qt"]))
    ref_rule = oracle.sage_emulate(g["qi"], g["ki"], g["vt"], g["qs"], g["ks"], g["va"], S, S, H, H, 128,
                                   kv_valid=mk, rows=rows, headroom=0.0)
    exact = oracle.attention_f64(_bits(q), _bits(k), _bits(v), S, S, H, H, 128, kv_valid=mk, rows=rows)
    got = _f32(o[torch.from_numpy(rows).long().to(cuda)])
    c_emu, c_ex, rr = cosine(got, emu), cosine(got, exact), rel_rms(got, exact)
    rr_ref = rel_rms(ref_rule, exact)
    print(f"config3 q_group=64: cos(emu)={c_emu:.7f} cos(exact)={c_ex:.6f} relrms={rr:.4f} "
          f"relrms(reference rule)={rr_ref:.4f}", flush=True)
    # the gate of _sage_vs_oracle: 4 %, or the reference arithmetic's own figure + 0.25 points
    assert c_emu >= 0.99999 and c_ex >= 0.995 and rr < max(0.04, rr_ref + 0.0025)


@pytest.mark.parametrize("Sq,Skv,Hq,Hkv,D,pad", [(300, 300, 4, 4, 128, 0), (130, 517, 4, 2, 128, 8),
                                              (64, 64, 2, 2, 128, 0), (130, 517, 4, 2, 64, 8)])
def test_q_group_64_prologue_bit_exact(cuda, Sq, Skv, Hq, Hkv, D, pad):
    """Q per 64 tokens on small shapes: a partial last 64-row block (rows past Sq count
    as zeros), GQA, padded strides; every workspace region against the oracle with G = 64."""
    print(f"q_group=64 prologue {Sq}x{Skv} H={Hq}/{Hkv} pad={pad}", flush=True)
    q, k, v, qs, ks = _bias_inputs(Sq, Skv, Hq, Hkv, D, pad, 2.0, cuda, Sq * 13 + Skv)
    p = AttnParams(Sq=Sq, Skv=Skv, Hq=Hq, Hkv=Hkv, D=D, q_stride=qs, kv_stride=ks, o_stride=qs)
    ws = _ws(p, cuda)
    sage_quantize(q, k, v, p, ws, q_group=64)
    torch.cuda.synchronize()
    g = _quantized(ws, p, sage_layout(p))
    _, want = oracle.sage_reference(_bits(q), _bits(k), _bits(v), Sq, Skv, Hq, Hkv, D, q_stride=qs, kv_stride=ks,
                                    q_group=64, rows=np.zeros(0, np.int32))
    want["qs"] = np.repeat(want["qs"], 4, axis=1)
    for name in ("km", "va", "qs", "ks", "qi", "ki", "vt"):
        assert np.array_equal(g[name], want[name]), name


def _sage_vs_oracle(cuda, q, k, v, mask, S, H, rows, seed_note=""):
    p = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=128, kv_valid=mask)
    ws = _ws(p, cuda)
    o = torch.empty_like(q)
    flash_attn_fp8(q, k, v, o, p, ws)
    # the quantized operands the emulator is fed: flash_attn_fp8 quantizes Q inside the
    # attention kernel (the workspace holds no Q), bit-identical to the prologue's Q
    # (test_fused_q_equals_prologue_q), which sage_quantize writes
    wsq = _ws(p, cuda)
    sage_quantize(q, k, v, p, wsq)
    torch.cuda.synchronize()
    L = sage_layout(p)
    g = _quantized(wsq, p, L)
    rows = np.array(rows, np.int32)
    mk = None if mask is None else mask.cpu().numpy()
    # the kernel balances its grid by splitting the last round's units by key range;
    # the emulator follows the same plan
    units = (S + L["split_qt"] - 1) // L["split_qt"] * H
    emu = oracle.sage_emulate(g["qi"], g["ki"], g["vt"], g["qs"], g["ks"], g["va"], S, S, H, H, 128,
                              kv_valid=mk, rows=rows, headroom=oracle.KERNEL_HEADROOM,
                              split=(units - L["split_units"], L["split_parts"], L["split_qt"]))
    ref_rule = oracle.sage_emulate(g["qi"], g["ki"], g["vt"], g["qs"], g["ks"], g["va"], S, S, H, H, 128,
                                   kv_valid=mk, rows=rows, headroom=0.0)
    exact = oracle.attention_f64(_bits(q), _bits(k), _bits(v), S, S, H, H, 128, kv_valid=mk, rows=rows)
    # the kernel's lazy-max rule is no less accurate than the reference's exact-max rule
    # (they differ by fp8 rounding of P, so they are compared through the exact result)
    assert rel_rms(emu, exact) <= 1.1 * rel_rms(ref_rule, exact) + 1e-3
    got = _f32(o[torch.from_numpy(rows).long().to(cuda)])
    c_emu, e_emu = cosine(got, emu), max_abs(got, emu)
    c_ex, rr = cosine(got, exact), rel_rms(got, exact)
    rr_ref = rel_rms(ref_rule, exact)
    h2 = oracle.sage_emulate(g["qi"], g["ki"], g["vt"], g["qs"], g["ks"], g["va"], S, S, H, H, 128,
                             kv_valid=mk, rows=rows, headroom=2.0)
    print(f"{seed_note} sage: cos(emu)={c_emu:.7f} maxabs(emu)={e_emu:.3g} cos(exact)={c_ex:.6f} relrms={rr:.4f} "
          f"relrms(emulator H=0 reference rule / H=2 / H=3 kernel rule)={rr_ref:.4f} / {rel_rms(h2, exact):.4f} / "
          f"{rel_rms(emu, exact):.4f}", flush=True)
    # emulator fed the same workspace: accumulation order and the bf16 store differ, and
    # the GPU's exp2 (v_exp_f32, within 1 ulp) against libm's can move a probability across
    # an e4m3 rounding boundary, one e4m3 step (2^-4 relative) of that key's weight
    assert c_emu >= 0.99999 and e_emu <= max(2e-2, 2.0 ** -4 * np.abs(emu).max())
    # Cosine >= 0.995 against exact attention, and the reference's 4 % rel-RMS gate
    # (tests/attention_fp8_test.cpp:65) unless the reference's own arithmetic (exact-max
    # emulator on the same quantized operands) already exceeds it on this input: then
    # the kernel is held to that figure plus 0.1 points (the lazy max's 2^-3 scaling of P
    # gives up three binades of e4m3's normal range at the small-weight end).
    assert c_ex >= 0.995
    assert rr < max(0.04, rr_ref + 0.001), (rr, rr_ref)
    return o


@pytest.mark.parametrize("cfg_id", [1, 3, 4, 5])
def test_sage_configs(cuda, cfg_id):
    cfg = CONFIGS[cfg_id]
    print(f"config {cfg_id} {cfg.name}", flush=True)
    q, k, v, mask = make_inputs(cfg, seed=cfg_id, device=cuda)
    rows = sorted(set(query_rows(cfg.S, cfg.H)) | set(range(0, cfg.S, max(1, cfg.S // 40))))
    _sage_vs_oracle(cuda, q, k, v, mask, cfg.S, cfg.H, rows, f"config{cfg_id}")


@pytest.mark.parametrize("Sq,Skv,Hq,Hkv,D,pad,kbias", [
    (300, 300, 4, 4, 128, 0, 0.0), (257, 1000, 4, 2, 128, 0, 4.0), (130, 77, 2, 2, 64, 8, 2.0),
    (1024, 4352, 2, 2, 128, 0, 8.0),
])
def test_reference_sage_cases(cuda, Sq, Skv, Hq, Hkv, D, pad, kbias):
    """The reference's four Sage cases (tests/attention_fp8_test.cpp:110-113), D = 64
    included, all on the quantized path: rel-RMS < 4 % against exact attention."""
    q, k, v, qs, ks = _bias_inputs(Sq, Skv, Hq, Hkv, D, pad, kbias, cuda, Sq * 31 + Skv)
    p = AttnParams(Sq=Sq, Skv=Skv, Hq=Hq, Hkv=Hkv, D=D, q_stride=qs if pad else 0, kv_stride=ks if pad else 0,
                   o_stride=qs if pad else 0)
    assert flash_attn_fp8_ok(q, k, v, q, p)
    ws = _ws(p, cuda)
    o = torch.zeros(Sq * qs, dtype=torch.bfloat16, device=cuda)
    flash_attn_fp8(q, k, v, o, p, ws)
    torch.cuda.synchronize()
    exact = oracle.attention_f64(_bits(q), _bits(k), _bits(v), Sq, Skv, Hq, Hkv, D, q_stride=qs, kv_stride=ks)
    got = _f32(o.view(Sq, qs)[:, : Hq * D]).reshape(exact.shape)
    assert rel_rms(got, exact) < 0.04


def test_fallbacks_and_aliasing(cuda):
    S, H = 200, 2
    q, k, v, qs, ks = _bias_inputs(S, S, H, H, 128, 0, 1.0, cuda, 9)
    p = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=128)
    ref = torch.empty_like(q)
    flash_attn(q, k, v, ref, p)
    # no workspace -> flash_attn, bit for bit
    o = torch.empty_like(q)
    flash_attn_fp8(q, k, v, o, p, None)
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int16), ref.view(torch.int16))
    # causal or negative scale -> not the quantized path
    assert flash_attn_fp8_ok(q, k, v, o, p)
    assert not flash_attn_fp8_ok(q, k, v, o, AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=128, causal=1))
    assert not flash_attn_fp8_ok(q, k, v, o, AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=128, scale=-0.1))
    assert flash_attn_fp8_ok(q, k, v, o, AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=64))
    assert not flash_attn_fp8_ok(q, k, v, o, AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=72))
    # o aliasing q: same result as a separate output
    ws = _ws(p, cuda)
    sep = torch.empty_like(q)
    flash_attn_fp8(q, k, v, sep, p, ws)
    qa = q.clone()
    flash_attn_fp8(qa, k, v, qa, p, ws)
    torch.cuda.synchronize()
    assert torch.equal(qa.view(torch.int16), sep.view(torch.int16))
    # o aliasing q on a layout whose grid is split (config 3's shape): the split
    # parts and the last-arrival merge still read every Q row before any output row
    # of the unit is written
    cfg = CONFIGS[3]
    q3, k3, v3, m3 = make_inputs(cfg, seed=19, device=cuda)
    p3 = AttnParams(Sq=cfg.S, Skv=cfg.S, Hq=cfg.H, Hkv=cfg.H, D=128, kv_valid=m3)
    assert sage_layout(p3)["split_parts"] > 1
    ws3 = _ws(p3, cuda)
    sep3 = torch.empty_like(q3)
    flash_attn_fp8(q3, k3, v3, sep3, p3, ws3)
    flash_attn_fp8(q3, k3, v3, q3, p3, ws3)
    torch.cuda.synchronize()
    assert torch.equal(q3.view(torch.int16), sep3.view(torch.int16))
    # misaligned workspace is rejected
    with pytest.raises(RuntimeError, match="256-byte aligned"):
        flash_attn_fp8(q, k, v, o, p, ws.data_ptr() + 16)


def test_sage_mask_equals_compacted_keys(cuda):
    """Masked Sage == Sage over the compacted keys, up to quantization-grid effects
    (K groups and the K mean shift with compaction), at config-2 size."""
    cfg = CONFIGS[2]
    q, k, v, mask = make_inputs(cfg, seed=22, device=cuda)
    S, H = cfg.S, cfg.H
    o1 = torch.empty_like(q); o2 = torch.empty_like(q)
    p1 = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=128, kv_valid=mask)
    flash_attn_fp8(q, k, v, o1, p1, _ws(p1, cuda))
    sel = mask.bool()
    kc, vc = k[sel].contiguous(), v[sel].contiguous()
    p2 = AttnParams(Sq=S, Skv=int(sel.sum()), Hq=H, Hkv=H, D=128)
    flash_attn_fp8(q, kc, vc, o2, p2, _ws(p2, cuda))
    torch.cuda.synchronize()
    assert cosine(_f32(o1), _f32(o2)) > 0.999


def test_split_units_dead_parts_and_repeat(cuda):
    """Key-range split of the grid's last round: a unit whose first parts see only
    padded keys merges to the same result as exact attention over the valid keys,
    and repeated calls on one workspace are bit-identical (the arrival counters
    return to zero after every merge)."""
    Sq, Skv, H = 1024, 4352, 2
    q, k, v, qs, ks = _bias_inputs(Sq, Skv, H, H, 128, 0, 2.0, cuda, 77)
    mask = torch.ones(Skv, dtype=torch.uint8, device=cuda)
    mask[: Skv * 2 // 5] = 0  # the first 40 % of the keys: whole parts with no live key
    p = AttnParams(Sq=Sq, Skv=Skv, Hq=H, Hkv=H, D=128, kv_valid=mask)
    L = sage_layout(p)
    print(f"split units {L['split_units']} parts {L['split_parts']}", flush=True)
    # fewer units than work-group slots: every unit is split, into the most parts
    assert L["split_units"] == (Sq + L["split_qt"] - 1) // L["split_qt"] * H and L["split_parts"] == 4
    ws = _ws(p, cuda)
    outs = []
    for _ in range(3):
        o = torch.empty_like(q)
        flash_attn_fp8(q, k, v, o, p, ws)
        outs.append(o)
    torch.cuda.synchronize()
    assert all(torch.equal(outs[0].view(torch.int16), x.view(torch.int16)) for x in outs[1:])
    exact = oracle.attention_f64(_bits(q), _bits(k), _bits(v), Sq, Skv, H, H, 128, kv_valid=mask.cpu().numpy())
    got = _f32(outs[0]).reshape(exact.shape)
    assert cosine(got, exact) >= 0.995 and rel_rms(got, exact) < 0.04


def test_split_repeat_across_shapes(cuda):
    """Two split plans sharing one workspace in alternation (config 3: 304 units x 3
    parts after a full round; 2048 x 8 heads: all 128 units x 2 parts, the partial
    regions overlap): every call of a shape reproduces that shape's first output bit
    for bit, so no call reads partials or counters another call left behind."""
    outs, ins = {}, {}
    ws = None
    c = CONFIGS[3]
    q, k, v, m = make_inputs(c, seed=3, device=cuda)
    ins[3] = (q, k, v, AttnParams(Sq=c.S, Skv=c.S, Hq=c.H, Hkv=c.H, D=128, kv_valid=m))
    q, k, v, *_ = _bias_inputs(2048, 2048, 8, 8, 128, 0, 2.0, cuda, 41)
    ins["2048x8"] = (q, k, v, AttnParams(Sq=2048, Skv=2048, Hq=8, Hkv=8, D=128))
    for cid, (q, k, v, p) in ins.items():
        L = sage_layout(p)
        print(f"{cid}: split units {L['split_units']} parts {L['split_parts']}", flush=True)
        assert L["split_parts"] > 1
        n = flash_attn_fp8_workspace(p)
        ws = n if ws is None else max(ws, n)
    ws = torch.empty(ws, dtype=torch.uint8, device=cuda)
    for rep in range(3):
        for cid in ins:
            q, k, v, p = ins[cid]
            o = torch.empty_like(q)
            flash_attn_fp8(q, k, v, o, p, ws)
            torch.cuda.synchronize()
            if rep == 0:
                outs[cid] = o
            else:
                assert torch.equal(o.view(torch.int16), outs[cid].view(torch.int16)), (cid, rep)


@pytest.mark.parametrize("Sq,Skv,Hq,Hkv,pad,kbias,masked", [
    (130, 77, 2, 2, 8, 2.0, False), (130, 77, 2, 2, 5, 2.0, False), (300, 300, 4, 4, 0, 0.0, False),
    (257, 1000, 4, 2, 0, 4.0, True),
    (4352, 4352, 24, 24, 0, 8.0, True),
])
def test_sage_d64(cuda, Sq, Skv, Hq, Hkv, pad, kbias, masked):
    """Sage at D = 64 (the reference's run<64>, attention_fp8.cu:496-497): the kernel
    against the emulator fed the same workspace and against exact attention, under the
    gate of _sage_vs_oracle. The last shape has 408 units of 256 queries, so the
    grid's last round is split by key range and merged."""
    D = 64
    print(f"sage D=64 {Sq}x{Skv} H={Hq}/{Hkv} pad={pad} masked={masked}", flush=True)
    q, k, v, qs, ks = _bias_inputs(Sq, Skv, Hq, Hkv, D, pad, kbias, cuda, Sq * 7 + Skv)
    mask = None
    if masked:
        g = torch.Generator().manual_seed(Skv)
        mask = (torch.rand(Skv, generator=g) > 0.2).to(torch.uint8).to(cuda)
    p = AttnParams(Sq=Sq, Skv=Skv, Hq=Hq, Hkv=Hkv, D=D, q_stride=qs, kv_stride=ks, o_stride=qs, kv_valid=mask)
    assert flash_attn_fp8_ok(q, k, v, q, p)
    L = sage_layout(p)
    ws = _ws(p, cuda)
    o = torch.zeros_like(q)
    flash_attn_fp8(q, k, v, o, p, ws)
    torch.cuda.synchronize()
    g = _quantized(ws, p, L)
    mk = None if mask is None else mask.cpu().numpy()
    rows = np.array(sorted(set(query_rows(Sq, Hq)) | set(range(0, Sq, max(1, Sq // 40)))), np.int32)
    units = (Sq + L["split_qt"] - 1) // L["split_qt"] * Hq
    if Sq == 4352:
        assert L["split_units"] > 0
    emu = oracle.sage_emulate(g["qi"], g["ki"], g["vt"], g["qs"], g["ks"], g["va"], Sq, Skv, Hq, Hkv, D,
                              kv_valid=mk, rows=rows, headroom=oracle.KERNEL_HEADROOM,
                              split=(units - L["split_units"], L["split_parts"], L["split_qt"]))
    ref_rule = oracle.sage_emulate(g["qi"], g["ki"], g["vt"], g["qs"], g["ks"], g["va"], Sq, Skv, Hq, Hkv, D,
                                   kv_valid=mk, rows=rows, headroom=0.0)
    exact = oracle.attention_f64(_bits(q), _bits(k), _bits(v), Sq, Skv, Hq, Hkv, D, q_stride=qs, kv_stride=ks,
                                 kv_valid=mk, rows=rows)
    got = _f32(o.view(Sq, qs)[torch.from_numpy(rows).long().to(cuda), : Hq * D]).reshape(exact.shape)
    c_emu, e_emu = cosine(got, emu), max_abs(got, emu)
    c_ex, rr, rr_ref = cosine(got, exact), rel_rms(got, exact), rel_rms(ref_rule, exact)
    print(f"  cos(emu)={c_emu:.7f} maxabs(emu)={e_emu:.3g} cos(exact)={c_ex:.6f} relrms={rr:.4f} "
          f"relrms(reference rule)={rr_ref:.4f}", flush=True)
    assert c_emu >= 0.99999 and e_emu <= max(2e-2, 2.0 ** -4 * np.abs(emu).max())  # as _sage_vs_oracle
    assert c_ex >= 0.995 and rr < max(0.04, rr_ref + 0.0025)


# flash_attn_fp8 on the D = 128 pipe kernel quantizes Q inside the attention kernel
# (the prologue skips it); sage_quantize + sage_attend quantize Q in the prologue.
# Both must give the same output bit for bit: ragged and padded query rows, GQA,
# masks, a negative-free scale other than the default, split grids, config 3.
# Sq, Skv, Hq, Hkv, pad, kbias, scale, masked
FUSED_Q = [
    (1, 64, 1, 1, 0, 1.0, 0.0, False), (77, 300, 4, 2, 5, 2.0, 0.0, True), (1000, 1117, 6, 3, 8, 4.0, 0.3, False),
    (2047, 2047, 4, 4, 0, 1.0, 0.0, True), (4352, 4352, 24, 24, 0, 2.0, 0.0, True),
]


@pytest.mark.parametrize("case", FUSED_Q, ids=lambda c: "x".join(map(str, c[:4])) + f"_p{c[4]}{'_m' if c[7] else ''}")
def test_fused_q_equals_prologue_q(cuda, case):
    Sq, Skv, Hq, Hkv, pad, kbias, scale, masked = case
    print(f"fused-Q case {case}", flush=True)
    q, k, v, qs, ks = _bias_inputs(Sq, Skv, Hq, Hkv, 128, pad, kbias, cuda, 31 + Sq)
    mask = None
    if masked:
        mask = (torch.rand(Skv, generator=torch.Generator().manual_seed(Skv)) > 0.1).to(torch.uint8).to(cuda)
    p = AttnParams(Sq=Sq, Skv=Skv, Hq=Hq, Hkv=Hkv, D=128, scale=scale, q_stride=qs if pad else 0,
                   kv_stride=ks if pad else 0, kv_valid=mask)
    assert flash_attn_fp8_ok(q, k, v, q, p)
    ws1, ws2 = _ws(p, cuda), _ws(p, cuda)
    o1 = torch.full((Sq, Hq * 128), 3.0, dtype=torch.bfloat16, device=cuda)
    o2 = torch.full((Sq, Hq * 128), 5.0, dtype=torch.bfloat16, device=cuda)
    flash_attn_fp8(q, k, v, o1, p, ws1)
    sage_quantize(q, k, v, p, ws2)
    sage_attend(o2, p, ws2)
    torch.cuda.synchronize()
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    # K / V regions of the two workspaces agree as well (the prologue's K/V part is shared)
    L = sage_layout(p)
    a, b = _quantized(ws1, p, L), _quantized(ws2, p, L)
    for name in ("ki", "vt", "ks", "km", "va"):
        assert np.array_equal(a[name], b[name]), name

"""CPU-side checks of the C ABI: the library loads, exports every symbol the header
declares, rejects the reference's invalid inputs before touching a device, and
computes workspace sizes/layouts on the host. No kernel is launched here."""
import ctypes
import math
import os
import re

import pytest

from miroxen_amd import _lib
from miroxen_amd.attention import AttnParams, flash_attn, attn_reference, flash_attn_fp8_workspace, sage_layout

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "miroxen_attn.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"\b(mx_[a-z0-9_]+)\s*\(", src))


def test_header_and_binding_agree():
    assert _declared() == set(_lib.SYMBOLS)


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    for name in _declared():
        assert hasattr(L, name), name
    assert "gfx950" in L.mx_version().decode()


def test_library_imports_no_allocation_or_sync_api():
    """The reference's entry points do pure launches (attention.cu:411-458): no
    allocation, no host synchronisation. The library holds its split partials and the
    no-alloc scratch in fixed device arrays, so its dynamic imports contain no
    allocating, freeing or synchronising HIP call at all."""
    import shutil
    import subprocess
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--undefined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    imported = {line.split()[-1].split("@")[0] for line in out.splitlines() if line.strip()}
    hip = sorted(n for n in imported if n.startswith("hip"))
    assert "hipLaunchKernel" in hip
    bad = [n for n in hip if re.search(r"Malloc|Free|Alloc|Synchronize|hipMemcpy(?!.*Async)|hipMemset(?!.*Async)",
                                       n)]
    assert not bad, bad


def test_struct_layout_matches_header():
    # int x5, float, int x2, int64 x3, pointer: 8 4-byte fields = 32 bytes, then 3*8 + 8
    assert ctypes.sizeof(_lib.CParams) == 32 + 24 + 8
    assert _lib.CParams.q_stride.offset == 32


def _good():
    return AttnParams(Sq=1, Skv=1, Hq=1, Hkv=1, D=64)


# The reference's 11 invalid parameter sets x {flash_attn, attn_reference} + null q
# (tests/attention_test.cu:178-208): 23 rejections.
INVALID = [
    dict(Sq=0), dict(Skv=-1), dict(Hq=3, Hkv=2), dict(D=80), dict(causal=2), dict(Hkv=0),
    dict(q_stride=63), dict(kv_stride=-1), dict(o_stride=63), dict(scale=math.nan),
    dict(kv_stride=2 ** 63 - 1),
]


@pytest.mark.parametrize("i", range(len(INVALID)))
@pytest.mark.parametrize("fn", [flash_attn, attn_reference])
def test_invalid_params_rejected(fn, i):
    p = _good()
    for key, val in INVALID[i].items():
        setattr(p, key, val)
    dummy = 256  # any non-null address: validation fails before it is used
    with pytest.raises(RuntimeError):
        fn(dummy, dummy, dummy, dummy, p, stream=0)


def test_null_query_rejected():
    with pytest.raises(RuntimeError, match="null tensor pointer"):
        flash_attn(0, 256, 256, 256, _good(), stream=0)


def test_error_message_is_reference_text():
    p = _good(); p.D = 80
    with pytest.raises(RuntimeError, match="unsupported head dimension 80"):
        flash_attn(256, 256, 256, 256, p, stream=0)


def test_too_many_heads_rejected():
    p = AttnParams(Sq=1, Skv=1, Hq=65536, Hkv=1, D=128)
    with pytest.raises(RuntimeError, match="too many heads"):
        flash_attn(256, 256, 256, 256, p, stream=0)


def test_workspace_and_layout():
    assert flash_attn_fp8_workspace(AttnParams()) == 0
    p = AttnParams(Sq=4352, Skv=4352, Hq=24, Hkv=24, D=128)
    L = sage_layout(p)
    assert L["sq_pad"] == 4352 and L["skv_pad"] == 4352
    for name in ("qi", "ki", "vt", "qs", "ks", "km", "va", "part", "split", "cnt", "total"):
        assert L[name] % 256 == 0
    assert L["qi"] == 0 and L["ki"] == 24 * 4352 * 128 and L["vt"] == 2 * 24 * 4352 * 128
    assert flash_attn_fp8_workspace(p) == L["total"]
    # config 2: ~40 MB, plus one partial (fp16 normalised output, fp32 m, l per lane)
    # per split work-group;
    # the layout is a pure function of the shape (no device here): the pipelined kernel's
    # 128-query units, 816 on 512 work-group slots, the last 304 in three key ranges
    nw = L["split_qt"] // 32
    assert L["split_qt"] == 128 and L["split_units"] == 304 and L["split_parts"] == 3
    assert L["total"] < 45e6 + 4 * (nw * 2176) * L["split_units"] * L["split_parts"]
    assert L["cnt"] - L["split"] >= 4 * (nw * 2176) * L["split_units"] * L["split_parts"]
    # grids of one dispatch round (<= 512 units): split only where the parts spread over
    # idle CUs enough to pay for their merge (measured on the box, µs: 1088 x 24 heads
    # 18 unsplit / 22 in two parts; 2048 x 24: 42 / 45; 2048 x 8: 26 / 23; 1024 x 2: 4 parts)
    for (S, H), parts in {(1088, 24): 1, (2048, 24): 1, (512, 24): 1, (2048, 8): 2, (1024, 2): 4}.items():
        Lp = sage_layout(AttnParams(Sq=S, Skv=S if S != 1024 else 4352, Hq=H, Hkv=H, D=128))
        assert Lp["split_parts"] == parts, (S, H, Lp["split_parts"])
        units = (S + 127) // 128 * H
        assert Lp["split_units"] == (units if parts > 1 else 0)
    # the D = 64 kernel (256-query units, one work-group per CU): 2048 x 24 heads 39 us
    # unsplit against 44 in four parts; 1088 x 24: 21 in two parts against 23 unsplit
    for (S, H), parts in {(2048, 24): 1, (1088, 24): 2}.items():
        assert sage_layout(AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=64))["split_parts"] == parts, (S, H)
    p2 = AttnParams(Sq=1000, Skv=77, Hq=4, Hkv=2, D=128)
    L2 = sage_layout(p2)
    assert L2["sq_pad"] == 1024 and L2["skv_pad"] == 128
    order = [L2[n] for n in ("qi", "ki", "vt", "qs", "ks", "km", "va", "part", "split", "cnt", "total")]
    assert order == sorted(order)
    assert L2["ki"] - L2["qi"] >= 4 * 1024 * 128 and L2["vt"] - L2["ki"] >= 2 * 128 * 128


def test_cpp_dropin_header_rejects_invalid_inputs(tmp_path):
    """Compile the reference-style invalid-input test against include/miroxen/attention.h
    and libmiroxen_attn.so, and run it (host-side validation only, no GPU needed)."""
    import subprocess
    exe = tmp_path / "invalid_inputs"
    lib_dir = os.path.dirname(_lib.LIB_PATH)
    cmd = ["/opt/rocm/bin/hipcc", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "cpp", "invalid_inputs.cpp"), "-L", lib_dir, "-lmiroxen_attn",
           f"-Wl,-rpath,{lib_dir}", "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "23 rejected" in r.stdout and "blockscale 10/10 ok" in r.stdout


@pytest.mark.parametrize("bad", [dict(D=7), dict(D=258), dict(rot=130), dict(rot=3), dict(mode=3),
                                 dict(cos=0), dict(H=0), dict(col0=-1)])
def test_head_norm_rope_rejects(bad):
    """Reference MX_CHECK (src/kernels/ops.cu:201) plus null/shape checks, host-side."""
    from miroxen_amd import head_norm_rope
    a = dict(S=4, in_stride=256, col0=0, H=2, D=128, rot=128, mode=1, cos=256, sin=256)
    a.update(bad)
    with pytest.raises(RuntimeError):
        head_norm_rope(256, a["S"], a["in_stride"], a["col0"], a["H"], a["D"], None, 1e-6, a["cos"], a["sin"],
                       a["rot"], a["mode"], 512, stream=0)


def test_sage_tile_loop_is_generated():
    """The committed inline-assembly tile loop (sage_tile.inc) is the generator's
    output; the generator also asserts its hazard distances while emitting it."""
    import importlib.util
    src = os.path.join(ROOT, "miroxen_amd", "csrc", "gen_sage_tile.py")
    spec = importlib.util.spec_from_file_location("gen_sage_tile", src)
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    with open(os.path.join(ROOT, "miroxen_amd", "csrc", "sage_tile.inc")) as f:
        assert f.read() == gen.generate()


def test_fp8_ok_rejects_keys_past_32bit_offsets():
    """The quantized kernels address a K/V head through 32-bit buffer offsets: a head of
    skv_pad * D >= 2^32 bytes is not taken (the caller falls back to flash_attn). The
    decision is made before any device query, so it holds without a GPU."""
    from miroxen_amd.attention import flash_attn_fp8_ok
    for D, skv in ((128, 2 ** 25), (64, 2 ** 26), (128, 2 ** 25 + 1)):
        p = AttnParams(Sq=64, Skv=skv, Hq=1, Hkv=1, D=D)
        assert not flash_attn_fp8_ok(256, 256, 256, 256, p)


def test_workspace_layout_d64():
    """D = 64 runs the 8-wave kernel (256-query units): config-2 shape at D = 64 has 408
    units on 256 slots, so its last 152 units are split; the partials are sized for
    D = 64 (8 waves x (32 fp16 of output + fp32 m, l) x 64 lanes)."""
    p = AttnParams(Sq=4352, Skv=4352, Hq=24, Hkv=24, D=64)
    L = sage_layout(p)
    assert L["split_qt"] == 256 and L["split_units"] == 152 and L["split_parts"] > 1
    assert L["ki"] == 24 * 4352 * 64 and L["vt"] == 2 * 24 * 4352 * 64
    per_wg = 4 * (8 * 4 * 64 * 4 + 8 * 64 * 2)
    assert L["cnt"] - L["split"] >= per_wg * L["split_units"] * L["split_parts"]
    assert L["cnt"] - L["split"] < per_wg * L["split_units"] * L["split_parts"] + 256


def test_mfma_path_for_unaligned_strides():
    """flash_attn runs the MFMA kernel for token strides that are not multiples of 8
    elements (the reference's Aligned = false case) and for operands at 2-byte alignment;
    an odd (not bf16-aligned) address takes the general kernel. Host-side query."""
    from miroxen_amd.attention import flash_attn_uses_mfma
    base = 1 << 20
    for qs, ks in ((0, 0), (4 * 128 + 5, 2 * 128 + 7), (4 * 128 + 6, 2 * 128 + 8)):
        p = AttnParams(Sq=100, Skv=300, Hq=4, Hkv=2, D=128, q_stride=qs, kv_stride=ks, o_stride=qs)
        assert flash_attn_uses_mfma(base, base + 2, base + 6, base, p)
    p = AttnParams(Sq=100, Skv=300, Hq=4, Hkv=2, D=128)
    assert not flash_attn_uses_mfma(base + 1, base, base, base, p)


def test_flash_split_plan():
    """mx_flash_attn_split_plan on 256 CUs: grids of few units split by key range (up to
    8 parts of >= 4 tiles); the config-2 grid (408 units, a last round of 152 on a
    power-limited chip), whole rounds, causal calls and short key ranges run unsplit.
    Host-side."""
    from miroxen_amd.attention import flash_attn_split_plan
    P = lambda Sq, Skv, H, D=128, c=0: AttnParams(Sq=Sq, Skv=Skv, Hq=H, Hkv=H, D=D, causal=c)
    assert flash_attn_split_plan(P(4352, 4352, 24), 256) == (408, 0, 1)
    assert flash_attn_split_plan(P(4096, 4096, 32), 256) == (512, 0, 1)
    assert flash_attn_split_plan(P(1024, 8192, 8, c=1), 256) == (32, 0, 1)
    assert flash_attn_split_plan(P(300, 300, 2), 256) == (4, 0, 1)
    for shape in ((256, 2048, 2), (1000, 1000, 2), (4352, 4352, 6), (600, 2000, 6, 64), (1000, 1000, 4, 72)):
        f, u, s = flash_attn_split_plan(P(shape[0], shape[1], shape[2], *shape[3:]), 256)
        ntq = -(-shape[0] // 256)
        assert f == 0 and u == ntq * shape[2] and 2 <= s <= 8 and s * 4 <= -(-shape[1] // 64), (shape, f, u, s)
    # the plan depends on the CU count it is given: 1 CU runs every grid whole
    assert flash_attn_split_plan(P(256, 2048, 2), 1) == (2, 0, 1)

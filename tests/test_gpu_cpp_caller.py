"""The C++ drop-in header on the GPU: tests/cpp/attn_caller.cpp (built by
miroxen_amd.build.build_cpp_caller) calls mx::flash_attn and mx::flash_attn_fp8 from
include/miroxen/attention.h exactly as a reference DiT block does, at config 1
(H=24, S=1088, D=128). Its outputs must equal the Python binding's bit for bit (one
library, one path) and match the CPU oracle: exact attention for BF16 (cosine
>= 0.9999, max error <= 2e-2) and for Sage (cosine >= 0.995, rel-RMS < 4 %)."""
import os
import subprocess

import numpy as np
import pytest
import torch

import oracle
from miroxen_amd import AttnParams, flash_attn, flash_attn_fp8, flash_attn_fp8_workspace
from miroxen_amd.build import CPP_CALLER
from miroxen_amd.synth import CONFIGS, make_inputs
from tests.helpers import cosine, max_abs, query_rows, rel_rms

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def test_cpp_header_caller_config1(cuda, tmp_path):
    assert os.path.exists(CPP_CALLER), "tests/cpp/_build/attn_caller is not built (run __graft_entry__.build())"
    cfg = CONFIGS[1]
    S, H, D = cfg.S, cfg.H, cfg.D
    q, k, v, mask = make_inputs(cfg, seed=1, device=cuda)
    assert mask is None
    for name, t in (("q", q), ("k", k), ("v", v)):
        _bits(t).tofile(tmp_path / f"{name}.bin")
    print(f"C++ caller config 1: S={S} H={H} D={D}", flush=True)
    r = subprocess.run([CPP_CALLER, str(tmp_path), str(S), str(H), str(D), "0"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "fp8_ok 1" in r.stdout, r.stdout
    got_bf16 = np.fromfile(tmp_path / "o_bf16.bin", np.uint16)
    got_fp8 = np.fromfile(tmp_path / "o_fp8.bin", np.uint16)
    # the same calls through the Python binding
    p = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=D)
    o = torch.empty_like(q)
    flash_attn(q, k, v, o, p)
    ws = torch.empty(flash_attn_fp8_workspace(p), dtype=torch.uint8, device=cuda)
    o8 = torch.empty_like(q)
    flash_attn_fp8(q, k, v, o8, p, ws)
    torch.cuda.synchronize()
    assert np.array_equal(got_bf16, _bits(o).ravel())
    assert np.array_equal(got_fp8, _bits(o8).ravel())
    rows = np.array(sorted(set(query_rows(S, H)) | set(range(0, S, S // 40))), np.int32)
    exact = oracle.attention_f64(_bits(q), _bits(k), _bits(v), S, S, H, H, D, rows=rows)
    f32 = lambda h: oracle.bf16_to_f32(h).reshape(S, H, D)[rows]
    b, s8 = f32(got_bf16), f32(got_fp8)
    print(f"  bf16 cos={cosine(b, exact):.7f} maxabs={max_abs(b, exact):.3g}; "
          f"sage cos={cosine(s8, exact):.6f} relrms={rel_rms(s8, exact):.4f}", flush=True)
    assert cosine(b, exact) >= 0.9999 and max_abs(b, exact) <= 2e-2
    assert cosine(s8, exact) >= 0.995 and rel_rms(s8, exact) < 0.04

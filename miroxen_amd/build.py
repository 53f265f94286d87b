"""Build libmiroxen_attn.so (gfx950) in-tree with hipcc.

Usage: python -m miroxen_amd.build   (or __graft_entry__.build()).
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libmiroxen_attn.so")
SOURCES = ["blockscale.hip", "capi.hip", "flash_bf16.hip", "naive.hip", "norm_rope.hip", "sage.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # packed fp32 VALU ops stay off (device pass); the host pass warns it does not know the feature.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if c and (os.path.isabs(c) and os.path.exists(c) or not os.path.isabs(c)):
            return c
    return "hipcc"


def build(verbose: bool = False, out: str = LIB, defines=()) -> str:
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), "-I", CSRC,
           *[f"-D{d}" for d in defines], *[os.path.join(CSRC, s) for s in SOURCES], "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (r.stderr or "").splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{errs}")
    if verbose and errs.strip():
        print(errs)
    os.replace(tmp, out)
    return out


CPP_CALLER_SRC = os.path.join(ROOT, "tests", "cpp", "attn_caller.cpp")
CPP_CALLER = os.path.join(ROOT, "tests", "cpp", "_build", "attn_caller")


def build_cpp_caller(verbose: bool = False) -> str:
    """The C++ drop-in-header caller run by tests/test_gpu_cpp_caller.py (host code
    linked against libmiroxen_attn.so; built here so GPU runs need no compiler)."""
    os.makedirs(os.path.dirname(CPP_CALLER), exist_ok=True)
    cmd = [hipcc(), "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"), CPP_CALLER_SRC, "-L", LIBDIR,
           "-lmiroxen_attn", "-Wl,-rpath,$ORIGIN/../../../miroxen_amd/lib", "-o", CPP_CALLER]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{r.stderr}")
    return CPP_CALLER


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

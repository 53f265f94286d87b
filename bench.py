"""Benchmark of the DiT joint-attention hot path on one MI355X.

Workload (BASELINE.json metric "attention TFLOP/s + % MFMA peak at H=24,S=4352,D=128
(BF16 and Sage INT8/FP8)"): config 2, Qwen-Image 1024^2 joint attention, B=1, H=24,
S=4352, D=128, 200 of 256 text keys valid. A step is one attention call over that
batch with inputs resident in HBM. `value` is the BF16 flash kernel's TFLOP/s
(FLOP = 4*H*Sq*Skv*D, nominal Skv); the Sage INT8/FP8 path on config 3 (same shape,
K outlier channels) is reported in the same line under "sage", end to end including
its quantize prologue and kernel-only; the MXFP8 block-scaled GEMM of the DiT linears
(the reference's quoted M=8192 N=12288 K=4096) under "blockscale".

Prints ONE JSON line. --gpus above 1 is refused: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16 = 2500.0     # TFLOP/s, MI355X dense BF16 MFMA
PEAK_FP8 = 5000.0      # TFLOP/s, dense FP8 (INT8 5.0 POP/s)
PEAK_HBM = 8000.0      # GB/s


def _time(fn, steps: int, warmup: int, warm_s: float) -> float:
    """Average ms per call over `steps` calls, HIP events on the stream the kernels use
    (torch's current stream: the library launches on it). Warm-up: `warmup` calls and
    at least `warm_s` seconds of back-to-back calls, so the timed calls run at the
    GPU's sustained clock (it needs tens of ms of load to leave its idle clock state)."""
    import torch
    t0 = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t0 < warm_s:
        for _ in range(8):
            fn()
        n += 8
        torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(steps):
        fn()
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


MAX_GFX_MHZ = 2400.0  # MI355X maximum shader clock (the nominal peaks assume it)


class _Smi:
    """Board telemetry through amdsmi (the library behind amd-smi): per-XCD shader clock,
    the socket energy accumulator (15.3 uJ units) and the power-limit (PPT) residency
    counter. Absent or failing telemetry yields None; it never affects the timing."""

    def __init__(self):
        self.h = None
        try:
            import amdsmi
            amdsmi.amdsmi_init()
            self.smi = amdsmi
            self.h = amdsmi.amdsmi_get_processor_handles()[0]
            self.res = float(amdsmi.amdsmi_get_energy_count(self.h)["counter_resolution"])
        except Exception:
            self.h = None
            return
        self.board = {}
        try:
            self.board["power_limit_w"] = amdsmi.amdsmi_get_power_info(self.h)["power_limit"] / 1e6
            self.board["max_gfx_mhz"] = amdsmi.amdsmi_get_clock_info(self.h, amdsmi.AmdSmiClkType.GFX)["max_clk"]
        except Exception:
            pass

    def metrics(self):
        if self.h is None:
            return None
        try:
            return self.smi.amdsmi_get_gpu_metrics_info(self.h)
        except Exception:
            return None


_SMI = None


def _telemetry(fn, batch: int = 32, max_seconds: float = 3.0):
    """Shader clock and board power of one leg, from back-to-back calls of the leg's own
    call right after its timed region. The firmware refreshes the metrics table about
    once a second, so the window runs from the first refresh seen under load to the
    next one: power = energy-accumulator delta over the table's own timestamp delta
    (ns), clock = the per-XCD shader clocks of those refreshes (mean over XCDs and
    refreshes), ppt_residency = share of the window the firmware counted at the power
    limit."""
    import torch
    global _SMI
    if _SMI is None:
        _SMI = _Smi()
    first = _SMI.metrics()
    if first is None:
        return None
    snaps = []
    last_ts = first.get("system_clock_counter")
    t0 = time.perf_counter()
    while len(snaps) < 2 and time.perf_counter() - t0 < max_seconds:
        for _ in range(batch):
            fn()
        torch.cuda.synchronize()
        m = _SMI.metrics()
        if m is not None and m.get("system_clock_counter") != last_ts:
            last_ts = m.get("system_clock_counter")
            snaps.append(m)
    if len(snaps) < 2:
        return None
    a, b = snaps
    out = {}
    try:
        clocks = [x for m in snaps for x in m["current_gfxclks"] if isinstance(x, (int, float)) and x > 0]
        if clocks:
            out["gfx_mhz"] = round(sum(clocks) / len(clocks), 1)
        dts = (b["system_clock_counter"] - a["system_clock_counter"]) * 1e-9
        out["window_s"] = round(dts, 3)
        out["socket_w"] = round((b["energy_accumulator"] - a["energy_accumulator"]) * _SMI.res * 1e-6 / dts, 1)
        dacc = b["accumulation_counter"] - a["accumulation_counter"]
        if dacc > 0:
            out["ppt_residency"] = round((b["ppt_residency_acc"] - a["ppt_residency_acc"]) / dacc, 3)
    except (KeyError, TypeError, ZeroDivisionError):
        pass
    return out


def _at_clock(achieved: float, peak: float, tel) -> dict:
    """Roofline fraction against the peak scaled to the measured shader clock."""
    if not tel or "gfx_mhz" not in tel:
        return {}
    p = peak * tel["gfx_mhz"] / MAX_GFX_MHZ
    return {"peak_at_clock": round(p, 1), "frac_at_clock": round(achieved / p, 4)}


def _traffic(name: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (committed summary), or None."""
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("bytes_per_launch")


def cpu_baseline(q, k, v, mask, S, H, D, budget_s: float = 12.0):
    """The CPU oracle (C restatement of the reference's cpu_oracle, double accumulation,
    OpenMP over (row, head)) timed on a bounded sample of query rows of the same workload."""
    import numpy as np
    import torch

    import oracle
    threads = min(os.cpu_count() or 1, 16)
    bits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    qb, kb, vb = bits(q), bits(k), bits(v)
    mk = None if mask is None else mask.cpu().numpy()
    probe = np.arange(0, S, max(1, S // 16), dtype=np.int32)[:16]
    t0 = time.perf_counter()
    oracle.attention_f64(qb, kb, vb, S, S, H, H, D, kv_valid=mk, rows=probe, threads=threads)
    dt = max(time.perf_counter() - t0, 1e-3)
    n = int(min(S, max(16, len(probe) * budget_s / dt)))
    rows = np.linspace(0, S - 1, n).astype(np.int32)
    t0 = time.perf_counter()
    oracle.attention_f64(qb, kb, vb, S, S, H, H, D, kv_valid=mk, rows=rows, threads=threads)
    dt = time.perf_counter() - t0
    flop = 4.0 * H * n * S * D
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return {"value": round(flop / dt / 1e12, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "host_cpus": os.cpu_count(), "cpu_model": model,
            "sample": f"{n} of {S} query rows x {H} heads, all {S} keys, {dt:.1f} s; "
                      f"full call extrapolated {dt * S / n * 1e3:.0f} ms"}


def cpu_baseline_config1() -> dict:
    """The CPU oracle on config 1 (the reference's CPU-runnable case: H=24, S=1088, D=128,
    no mask) as a full call, every query row."""
    import numpy as np
    import torch

    import oracle
    from miroxen_amd.synth import CONFIGS, attn_flops, make_inputs
    c = CONFIGS[1]
    threads = min(os.cpu_count() or 1, 16)
    q, k, v, _ = make_inputs(c, seed=1)
    bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
    t0 = time.perf_counter()
    oracle.attention_f64(bits(q), bits(k), bits(v), c.S, c.S, c.H, c.H, c.D, threads=threads)
    dt = time.perf_counter() - t0
    return {"value": round(attn_flops(c.H, c.S, c.S, c.D) / dt / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "ms": round(dt * 1e3, 1),
            "sample": f"config 1 full call ({c.S} rows x {c.H} heads x {c.S} keys), {dt:.2f} s"}


def cpu_baseline_sage(q, k, v, mask, S, H, D, budget_s: float = 8.0) -> dict:
    """The Sage path on the CPU: the oracle's prologue (K mean, V abs-max, INT8 Q/K, e4m3
    V^T) over the whole config-3 input, then its emulator of the quantized kernel (exact
    int32 scores, e4m3 P, fp32 accumulation; OpenMP over (row, head)) on a bounded sample
    of query rows; the full call is the prologue plus the emulator extrapolated."""
    import numpy as np
    import torch

    import oracle
    threads = min(os.cpu_count() or 1, 16)
    bits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    qb, kb, vb = bits(q), bits(k), bits(v)
    mk = None if mask is None else mask.cpu().numpy()
    t0 = time.perf_counter()
    _, t = oracle.sage_reference(qb, kb, vb, S, S, H, H, D, kv_valid=mk, rows=np.zeros(0, np.int32),
                                 threads=threads)
    t_pro = time.perf_counter() - t0
    args = (t["qi"], t["ki"], t["vt"], t["qs"], t["ks"], t["va"], S, S, H, H, D)
    probe = np.arange(0, S, max(1, S // 16), dtype=np.int32)[:16]
    t0 = time.perf_counter()
    oracle.sage_emulate(*args, kv_valid=mk, rows=probe, threads=threads)
    dt = max(time.perf_counter() - t0, 1e-3)
    n = int(min(S, max(16, len(probe) * budget_s / dt)))
    rows = np.linspace(0, S - 1, n).astype(np.int32)
    t0 = time.perf_counter()
    oracle.sage_emulate(*args, kv_valid=mk, rows=rows, threads=threads)
    dt = time.perf_counter() - t0
    full = t_pro + dt * S / n
    flop = 4.0 * H * S * S * D
    return {"value": round(flop / full / 1e12, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"prologue over all {S} tokens {t_pro:.2f} s + emulator on {n} of {S} query rows x {H} "
                      f"heads, {dt:.1f} s; full call extrapolated {full * 1e3:.0f} ms"}


BS_M, BS_N, BS_K = 8192, 12288, 4096  # the reference's quoted block-scaled GEMM shape (src/kernels/blockscale.h:2)
BS_REF_TFLOPS = 152.0                 # its MXFP8 figure there (RTX 5060 Ti, cuBLASLt)
BS_REF_TFLOPS_FP4 = 293.0             # its NVFP4 figure there (src/kernels/blockscale.h:2)


def _blockscale_setup(dev, mode=None):
    """Block-scaled operands of the quoted shape (MXFP8 unless `mode`): W [N, K] quantized
    once, activations X [M, K]; returns the GEMM call Y[M, N] = X W^T (bf16 out)."""
    import torch

    from miroxen_amd.blockscale import QMat, QMode, gemm_blockscaled, qdata_bytes, qscale_bytes, quantize_blockscaled
    mode = QMode.MXFP8 if mode is None else mode
    g = torch.Generator(device=dev).manual_seed(41)
    x = torch.randn(BS_M, BS_K, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(BS_N, BS_K, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    mk = lambda r: QMat(torch.empty(qdata_bytes(mode, r, BS_K), dtype=torch.uint8, device=dev),
                        torch.empty(qscale_bytes(mode, r, BS_K), dtype=torch.uint8, device=dev),
                        torch.empty(4, dtype=torch.float32, device=dev))
    X, W = mk(BS_M), mk(BS_N)
    quantize_blockscaled(mode, w, BS_K, BS_N, BS_K, W)
    quantize_blockscaled(mode, x, BS_K, BS_M, BS_K, X)
    y = torch.empty(BS_M, BS_N, dtype=torch.bfloat16, device=dev)
    return lambda: gemm_blockscaled(mode, W, X, y, BS_N, BS_M, BS_N, BS_K)


def blockscale_cpu_baseline(budget_s: float = 8.0) -> dict:
    """The oracle's MXFP8 GEMM (C restatement: dequantize, double accumulation, OpenMP over
    output rows) timed on a bounded sample of X rows at the quoted shape, all of W."""
    import numpy as np

    import oracle
    threads = min(os.cpu_count() or 1, 16)
    rng = np.random.default_rng(41)
    wq = rng.integers(0, 0x7E, (BS_N, BS_K), dtype=np.uint8)
    ws = np.full((BS_N, BS_K // 32), 120, np.uint8)
    rows = 8
    xq = rng.integers(0, 0x7E, (rows, BS_K), dtype=np.uint8)
    xs = np.full((rows, BS_K // 32), 127, np.uint8)
    t0 = time.perf_counter()
    oracle.gemm_mxfp8(wq, ws, xq, xs, rows, BS_N, BS_K, threads=threads)
    dt = max(time.perf_counter() - t0, 1e-3)
    rows = int(min(512, max(8, rows * budget_s / dt)))
    xq = rng.integers(0, 0x7E, (rows, BS_K), dtype=np.uint8)
    xs = np.full((rows, BS_K // 32), 127, np.uint8)
    t0 = time.perf_counter()
    oracle.gemm_mxfp8(wq, ws, xq, xs, rows, BS_N, BS_K, threads=threads)
    dt = time.perf_counter() - t0
    flop = 2.0 * rows * BS_N * BS_K
    return {"value": round(flop / dt / 1e12, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{rows} of {BS_M} rows of X against all of W ({BS_N} x {BS_K}), {dt:.1f} s; "
                      f"full GEMM extrapolated {dt * BS_M / rows:.0f} s"}


def blockscale_leg(dev, steps: int, warmup: int, warm_s: float) -> dict:
    """MXFP8 block-scaled GEMM at the reference's quoted shape, and the activation
    quantizer at the reference's bench shapes (tests/blockscale_test.cpp:139), bytes
    counted as there: bf16 input + e4m3 output."""
    import torch

    from miroxen_amd.blockscale import QMat, QMode, qdata_bytes, qscale_bytes, quantize_blockscaled
    run = _blockscale_setup(dev)
    n = max(5, steps // 4)
    ms = _time(run, n, warmup, warm_s)
    tf = 2.0 * BS_M * BS_N * BS_K / (ms * 1e-3) / 1e12
    quant = {}
    for (M, K) in ((4096, 4096), (4096, 12288)):
        x = torch.randn(M, K, device=dev).to(torch.bfloat16)
        qm = QMat(torch.empty(qdata_bytes(QMode.MXFP8, M, K), dtype=torch.uint8, device=dev),
                  torch.empty(qscale_bytes(QMode.MXFP8, M, K), dtype=torch.uint8, device=dev))
        mq = _time(lambda: quantize_blockscaled(QMode.MXFP8, x, K, M, K, qm), steps, warmup, warm_s)
        gbs = (2.0 * M * K + M * K) / (mq * 1e-3) / 1e9
        quant[f"{M}x{K}"] = {"us": round(mq * 1e3, 2), "gbs": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM, 4)}
    # NVFP4: e2m1 data, e4m3 scale per 16, per-tensor amax; dequantized exactly to f16 in
    # the kernel and multiplied on the f16 MFMA (peak 2.5 PFLOP/s dense)
    run4 = _blockscale_setup(dev, QMode.NVFP4)
    ms4 = _time(run4, n, warmup, warm_s)
    tf4 = 2.0 * BS_M * BS_N * BS_K / (ms4 * 1e-3) / 1e12
    quant4 = {}
    for (M, K) in ((4096, 4096), (4096, 12288)):
        x = torch.randn(M, K, device=dev).to(torch.bfloat16)
        qm = QMat(torch.empty(qdata_bytes(QMode.NVFP4, M, K), dtype=torch.uint8, device=dev),
                  torch.empty(qscale_bytes(QMode.NVFP4, M, K), dtype=torch.uint8, device=dev),
                  torch.empty(4, dtype=torch.float32, device=dev))
        mq = _time(lambda: quantize_blockscaled(QMode.NVFP4, x, K, M, K, qm), steps, warmup, warm_s)
        gbs = (2.0 * M * K + M * K / 2) / (mq * 1e-3) / 1e9  # counted as the reference: bf16 in + fp4 out
        quant4[f"{M}x{K}"] = {"us": round(mq * 1e3, 2), "gbs": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM, 4)}
    nvfp4 = {"ms": round(ms4, 4), "tflops": round(tf4, 1), "reference_published_tflops": BS_REF_TFLOPS_FP4,
             "dtype": "e2m1 x e2m1 with e4m3 scales per 16, dequantized to f16 (exact), fp32 accumulate",
             "roofline": {"bound": "mfma", "achieved": round(tf4, 1), "peak": PEAK_BF16, "unit": "TFLOP/s",
                          "frac": round(tf4 / PEAK_BF16, 4), "traffic": _traffic("nvfp4_gemm")},
             "quantize": quant4}
    return {
        "workload": f"MXFP8 GEMM Y[M,N] = X[M,K] W[N,K]^T, M={BS_M} N={BS_N} K={BS_K}, bf16 out",
        "steps": n, "ms": round(ms, 4), "tflops": round(tf, 1),
        "reference_published_tflops": BS_REF_TFLOPS, "reference_hardware": "RTX 5060 Ti (cuBLASLt)",
        "dtype": "e4m3 x e4m3, UE8M0 scale per 32, fp32 accumulate",
        "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": PEAK_FP8, "unit": "TFLOP/s",
                     "frac": round(tf / PEAK_FP8, 4), "traffic": _traffic("mxfp8_gemm")},
        "quantize": quant,
        "nvfp4": nvfp4,
    }


def _only(which: str, n: int) -> int:
    """Run one kernel n times on the bench inputs (for rocprofv3 --pmc passes)."""
    import torch

    from miroxen_amd import AttnParams, flash_attn, flash_attn_fp8_workspace, sage_attend, sage_quantize
    from miroxen_amd.synth import CONFIGS, make_inputs
    dev = torch.device("cuda:0")
    if which == "copy":
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        for _ in range(n):
            b.copy_(a)
        torch.cuda.synchronize()
        return 0
    if which in ("blockscale", "nvfp4"):
        from miroxen_amd.blockscale import QMode
        run = _blockscale_setup(dev, QMode.NVFP4 if which == "nvfp4" else None)
        for _ in range(n):
            run()
        torch.cuda.synchronize()
        return 0
    cfg = CONFIGS[2 if which == "bf16" else 3]
    q, k, v, m = make_inputs(cfg, seed=2 if which == "bf16" else 3, device=dev)
    p = AttnParams(Sq=cfg.S, Skv=cfg.S, Hq=cfg.H, Hkv=cfg.H, D=cfg.D, kv_valid=m)
    o = torch.empty_like(q)
    ws = torch.empty(flash_attn_fp8_workspace(p), dtype=torch.uint8, device=dev)
    if which == "fused":  # fused norm/rope prologue on a [S, 3HD] projection (the bench's norm_rope_fused leg)
        from miroxen_amd import ROPE_INTERLEAVED, sage_quantize_norm_rope
        S, H, D = cfg.S, cfg.H, cfg.D
        g = torch.Generator(device=dev).manual_seed(33)
        t = torch.randn(S, 3 * H * D, device=dev, generator=g).to(torch.bfloat16)
        qw, kw = torch.rand(D, device=dev, generator=g) + 0.5, torch.rand(D, device=dev, generator=g) + 0.5
        ang = (torch.rand(S, D // 2, device=dev, generator=g) * 2 - 1) * 3.14159
        cs, sn = torch.cos(ang), torch.sin(ang)
        pr = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=D, q_stride=3 * H * D, kv_stride=3 * H * D, kv_valid=m)
        wsr = torch.empty(flash_attn_fp8_workspace(pr), dtype=torch.uint8, device=dev)
        b = t.data_ptr()
        for _ in range(n):
            sage_quantize_norm_rope(b, b + 2 * H * D, b + 4 * H * D, pr, qw, kw, 1e-6, cs, sn, D, ROPE_INTERLEAVED, wsr)
        torch.cuda.synchronize()
        return 0
    if which == "sage":
        sage_quantize(q, k, v, p, ws)
    from miroxen_amd import flash_attn_fp8
    for _ in range(n):
        if which == "bf16":
            flash_attn(q, k, v, o, p)
        elif which == "sage":
            sage_attend(o, p, ws)
        elif which == "sage_e2e":  # the product path: K/V prologue + attention quantizing Q
            flash_attn_fp8(q, k, v, o, p, ws)
        else:
            sage_quantize(q, k, v, p, ws)
    torch.cuda.synchronize()
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--warm-seconds", type=float, default=0.5,
                    help="minimum seconds of untimed back-to-back calls before each timed region")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--skip-large", action="store_true", help="skip configs 4 and 5 (S=12544, S=32760)")
    ap.add_argument("--no-blockscale", action="store_true", help="skip the MXFP8 block-scaled GEMM leg")
    ap.add_argument("--only", choices=["bf16", "sage", "sage_e2e", "prologue", "fused", "copy", "blockscale", "nvfp4"],
                    help="profiling driver: run just this kernel --steps times (no warm-up, no JSON); "
                         "'copy' is a 256 MiB device copy for calibrating HBM byte counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs the attention on one GPU only (no multi-GPU path); "
              "use --gpus 1", file=sys.stderr)
        return 2

    import torch

    if args.only:
        return _only(args.only, args.steps)

    from miroxen_amd import (ROPE_INTERLEAVED, ROPE_NONE, AttnParams, flash_attn, flash_attn_fp8,
                             flash_attn_fp8_workspace, head_norm_rope, sage_attend, sage_quantize,
                             sage_quantize_norm_rope, version)
    from miroxen_amd.synth import CONFIGS, attn_flops, make_inputs

    dev = torch.device("cuda:0")
    cfg = CONFIGS[2]
    S, H, D = cfg.S, cfg.H, cfg.D
    q, k, v, mask = make_inputs(cfg, seed=2, device=dev)
    p = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=D, kv_valid=mask)
    o = torch.empty_like(q)
    flop = attn_flops(H, S, S, D)
    eff_flop = attn_flops(H, S, int(mask.sum()), D)

    t0 = time.perf_counter()
    ms = _time(lambda: flash_attn(q, k, v, o, p), args.steps, args.warmup, args.warm_seconds)
    wall = time.perf_counter() - t0
    tflops = flop / (ms * 1e-3) / 1e12
    tel_bf16 = _telemetry(lambda: flash_attn(q, k, v, o, p))

    # ---- Sage INT8/FP8 on config 3 ----
    c3 = CONFIGS[3]
    q3, k3, v3, m3 = make_inputs(c3, seed=3, device=dev)
    p3 = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=D, kv_valid=m3)
    ws = torch.empty(flash_attn_fp8_workspace(p3), dtype=torch.uint8, device=dev)
    o3 = torch.empty_like(q3)
    ms_e2e = _time(lambda: flash_attn_fp8(q3, k3, v3, o3, p3, ws), args.steps, args.warmup, args.warm_seconds)
    ms_pro = _time(lambda: sage_quantize(q3, k3, v3, p3, ws), args.steps, args.warmup, args.warm_seconds)
    tel_e2e = _telemetry(lambda: flash_attn_fp8(q3, k3, v3, o3, p3, ws))
    ms_main = _time(lambda: sage_attend(o3, p3, ws), args.steps, args.warmup, args.warm_seconds)
    tel_main = _telemetry(lambda: sage_attend(o3, p3, ws))
    # config 3's stated Q grouping (one scale per 64-token block) beside the reference's 16
    ms_pro64 = _time(lambda: sage_quantize(q3, k3, v3, p3, ws, q_group=64), args.steps, args.warmup,
                     args.warm_seconds)

    def e2e64():
        sage_quantize(q3, k3, v3, p3, ws, q_group=64)
        sage_attend(o3, p3, ws)

    ms_e2e64 = _time(e2e64, args.steps, args.warmup, args.warm_seconds)
    pro_bytes = 9.0 * S * H * D  # read Q,K,V bf16 + write int8 Q, int8 K, fp8 V
    sage = {
        "workload": c3.name, "ms_end_to_end": round(ms_e2e, 4),
        "tflops_end_to_end": round(flop / (ms_e2e * 1e-3) / 1e12, 2),
        "ms_kernel": round(ms_main, 4), "tflops_kernel": round(flop / (ms_main * 1e-3) / 1e12, 2),
        "frac_fp8_peak_kernel": round(flop / (ms_main * 1e-3) / 1e12 / PEAK_FP8, 4),
        "speedup_vs_bf16_end_to_end": round(ms / ms_e2e, 3),
        "prologue_ms": round(ms_pro, 4), "prologue_gbs": round(pro_bytes / (ms_pro * 1e-3) / 1e9, 1),
        "prologue_frac_hbm": round(pro_bytes / (ms_pro * 1e-3) / 1e9 / PEAK_HBM, 4),
        "dtype": "int8 QK^T / e4m3 PV, fp32 accumulate",
        "q_group": 16,
        "q_group64": {"prologue_ms": round(ms_pro64, 4), "ms_end_to_end": round(ms_e2e64, 4),
                      "tflops_end_to_end": round(flop / (ms_e2e64 * 1e-3) / 1e12, 2)},
        "roofline": {"bound": "mfma", "achieved": round(flop / (ms_main * 1e-3) / 1e12, 2), "peak": PEAK_FP8,
                     "unit": "TFLOP/s", "frac": round(flop / (ms_main * 1e-3) / 1e12 / PEAK_FP8, 4),
                     "traffic": _traffic("sage_attn_config3"),
                     **_at_clock(flop / (ms_main * 1e-3) / 1e12, PEAK_FP8, tel_main)},
        "telemetry_end_to_end": tel_e2e, "telemetry_kernel": tel_main,
    }

    # ---- head_norm_rope fused into the Sage prologue (config-3 shape, Qwen-Image-style
    # interleaved RoPE over all 128 channels, per-head RMS-norm weights) ----
    # The reference's DiT block runs head_norm_rope on q, k and v (v: a plain dense copy,
    # ROPE_NONE) from the fused QKV projection, then the Sage prologue
    # (src/models/minimax_h3/dit.cpp:210-212, :223); the fused entry reads the projection once.
    g = torch.Generator(device=dev).manual_seed(33)
    HD = H * D
    t = torch.randn(S, 3 * HD, device=dev, generator=g).to(torch.bfloat16)
    qw = torch.rand(D, device=dev, generator=g) + 0.5
    kw = torch.rand(D, device=dev, generator=g) + 0.5
    ang = (torch.rand(S, D // 2, device=dev, generator=g) * 2 - 1) * 3.14159
    cs, sn = torch.cos(ang), torch.sin(ang)
    qd, kd, vd = (torch.empty(S, HD, dtype=torch.bfloat16, device=dev) for _ in range(3))
    pd = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=D, kv_valid=m3)
    pr = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=D, q_stride=3 * HD, kv_stride=3 * HD, o_stride=HD, kv_valid=m3)
    wsn = torch.empty(flash_attn_fp8_workspace(pr), dtype=torch.uint8, device=dev)
    base = t.data_ptr()

    def separate():
        head_norm_rope(t, S, 3 * HD, 0, H, D, qw, 1e-6, cs, sn, D, ROPE_INTERLEAVED, qd)
        head_norm_rope(t, S, 3 * HD, HD, H, D, kw, 1e-6, cs, sn, D, ROPE_INTERLEAVED, kd)
        head_norm_rope(t, S, 3 * HD, 2 * HD, H, D, None, 0.0, None, None, 0, ROPE_NONE, vd)
        sage_quantize(qd, kd, vd, pd, wsn)

    ms_sep = _time(separate, args.steps, args.warmup, args.warm_seconds)
    ms_fused = _time(lambda: sage_quantize_norm_rope(base, base + 2 * HD, base + 4 * HD, pr, qw, kw, 1e-6, cs, sn,
                                                     D, ROPE_INTERLEAVED, wsn),
                     args.steps, args.warmup, args.warm_seconds)
    ms_nr = _time(lambda: head_norm_rope(t, S, 3 * HD, 0, H, D, qw, 1e-6, cs, sn, D, ROPE_INTERLEAVED, qd),
                  args.steps, args.warmup, args.warm_seconds)
    nr_bytes = 4.0 * S * HD  # read + write bf16 of one [S, H, D] tensor
    sage["norm_rope_fused"] = {
        "ms_separate": round(ms_sep, 4), "ms_fused": round(ms_fused, 4),
        "speedup": round(ms_sep / ms_fused, 3),
        "fused_gbs": round(pro_bytes / (ms_fused * 1e-3) / 1e9, 1),
        "head_norm_rope_ms": round(ms_nr, 4), "head_norm_rope_gbs": round(nr_bytes / (ms_nr * 1e-3) / 1e9, 1),
        "chain": "separate = head_norm_rope x3 (q, k, v) + sage_quantize; fused = sage_quantize_norm_rope",
    }

    # ---- the other BASELINE configs at their full shapes (BF16 and Sage each) ----
    others = {}
    c1 = CONFIGS[1]
    q1, k1, v1, _ = make_inputs(c1, seed=1, device=dev)
    p1 = AttnParams(Sq=c1.S, Skv=c1.S, Hq=c1.H, Hkv=c1.H, D=c1.D)
    o1 = torch.empty_like(q1)
    w1 = torch.empty(flash_attn_fp8_workspace(p1), dtype=torch.uint8, device=dev)
    f1 = attn_flops(c1.H, c1.S, c1.S, c1.D)
    m1 = _time(lambda: flash_attn(q1, k1, v1, o1, p1), args.steps, args.warmup, args.warm_seconds)
    m1e = _time(lambda: flash_attn_fp8(q1, k1, v1, o1, p1, w1), args.steps, args.warmup, args.warm_seconds)
    others["config1"] = {"workload": c1.name, "H": c1.H, "S": c1.S, "steps": args.steps,
                         "bf16_ms": round(m1, 4), "bf16_tflops": round(f1 / (m1 * 1e-3) / 1e12, 1),
                         "sage_ms_end_to_end": round(m1e, 4),
                         "sage_tflops_end_to_end": round(f1 / (m1e * 1e-3) / 1e12, 1)}
    del q1, k1, v1, o1, w1
    if not args.skip_large:
        del q3, k3, v3, o3, ws, t, qd, kd, vd, wsn
        for cid in (4, 5):
            c = CONFIGS[cid]
            qc, kc, vc, mc = make_inputs(c, seed=cid, device=dev)
            pc = AttnParams(Sq=c.S, Skv=c.S, Hq=c.H, Hkv=c.H, D=c.D, kv_valid=mc)
            oc = torch.empty_like(qc)
            wc = torch.empty(flash_attn_fp8_workspace(pc), dtype=torch.uint8, device=dev)
            fc = attn_flops(c.H, c.S, c.S, c.D)
            n = max(3, args.steps // 20)
            mb = _time(lambda: flash_attn(qc, kc, vc, oc, pc), n, args.warmup, args.warm_seconds)
            me = _time(lambda: flash_attn_fp8(qc, kc, vc, oc, pc, wc), n, args.warmup, args.warm_seconds)
            # kernel-only: sage_attend reads the prologue's int8 Q, which flash_attn_fp8 (its
            # attention kernel quantizes Q itself) does not write
            sage_quantize(qc, kc, vc, pc, wc)
            mk = _time(lambda: sage_attend(oc, pc, wc), n, args.warmup, args.warm_seconds)
            tb = _telemetry(lambda: flash_attn(qc, kc, vc, oc, pc), batch=4)
            ts = _telemetry(lambda: sage_attend(oc, pc, wc), batch=4)
            others[f"config{cid}"] = {
                "workload": c.name, "H": c.H, "S": c.S, "steps": n,
                "bf16_ms": round(mb, 3), "bf16_tflops": round(fc / (mb * 1e-3) / 1e12, 1),
                "sage_ms_end_to_end": round(me, 3), "sage_tflops_end_to_end": round(fc / (me * 1e-3) / 1e12, 1),
                "sage_tflops_kernel": round(fc / (mk * 1e-3) / 1e12, 1),
                "telemetry_bf16": tb, "telemetry_sage_kernel": ts}
            del qc, kc, vc, oc, wc

    # ---- BF16 beyond the BASELINE configs: causal at config 2's shape (useful FLOP =
    # half the nominal), and grids of few units, where flash_attn splits the key range ----
    extras = {}
    if not args.skip_large:
        g = torch.Generator(device=dev).manual_seed(77)
        qx = torch.randn(S, H * D, device=dev, generator=g).to(torch.bfloat16)
        kx = torch.randn(S, H * D, device=dev, generator=g).to(torch.bfloat16)
        vx = torch.randn(S, H * D, device=dev, generator=g).to(torch.bfloat16)
        ox = torch.empty_like(qx)
        pcz = AttnParams(Sq=S, Skv=S, Hq=H, Hkv=H, D=D, causal=1)
        mc = _time(lambda: flash_attn(qx, kx, vx, ox, pcz), 50, args.warmup, args.warm_seconds)
        extras["bf16_causal_config2_shape"] = {"ms": round(mc, 4),
                                               "tflops_useful": round(flop / 2 / (mc * 1e-3) / 1e12, 1)}
        from miroxen_amd.attention import flash_attn_split_plan
        small = {}
        for sq, hh, skv in ((256, 2, 2048), (512, 4, 4096), (1024, 8, 8192)):
            qs_ = torch.randn(sq, hh * D, device=dev, generator=g).to(torch.bfloat16)
            ks_ = torch.randn(skv, hh * D, device=dev, generator=g).to(torch.bfloat16)
            vs_ = torch.randn(skv, hh * D, device=dev, generator=g).to(torch.bfloat16)
            os_ = torch.empty_like(qs_)
            ps = AttnParams(Sq=sq, Skv=skv, Hq=hh, Hkv=hh, D=D)
            msm = _time(lambda: flash_attn(qs_, ks_, vs_, os_, ps), 50, args.warmup, 0.1)
            small[f"{sq}x{hh}x{skv}"] = {"ms": round(msm, 4), "split_plan": list(flash_attn_split_plan(ps))}
        extras["bf16_small_grids"] = small
        del qx, kx, vx, ox

    bs = None if args.no_blockscale else blockscale_leg(dev, args.steps, args.warmup, args.warm_seconds)
    if bs is not None and not args.no_cpu:
        bs["cpu_baseline"] = blockscale_cpu_baseline()

    traffic = _traffic("flash_bf16_config2")
    line = {
        "metric": "attention TFLOP/s + % MFMA peak at H=24,S=4352,D=128 (BF16 and Sage INT8/FP8)",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded, config 2 distributions)",
        "config": {"workload": cfg.name, "B": 1, "H": H, "Sq": S, "Skv": S, "D": D,
                   "valid_keys": int(mask.sum()), "flop_nominal": flop, "flop_mask_effective": eff_flop,
                   "kernel": version()},
        "frac_bf16_peak": round(tflops / PEAK_BF16, 4),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_BF16, 4), "traffic": traffic,
                     **_at_clock(tflops, PEAK_BF16, tel_bf16)},
        "telemetry": tel_bf16,
        "board": getattr(_SMI, "board", None),
        "sage": sage,
        "other_configs": others,
        "extras": extras,
        "blockscale": bs,
        "timed_wall_s": round(wall, 3),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(q, k, v, mask, S, H, D)
        line["cpu_baseline_config1"] = cpu_baseline_config1()
        q3, k3, v3, m3 = make_inputs(c3, seed=3, device=dev)
        line["sage"]["cpu_baseline"] = cpu_baseline_sage(q3, k3, v3, m3, S, H, D)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

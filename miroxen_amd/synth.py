"""Seeded synthetic inputs for the five benchmark configurations.

Layout: q/k/v [S, H, D] bf16 token-major (reference src/kernels/attention.h:6-10),
kv_valid uint8 [S] or None. Joint sequences put the text slots first, then the
image/video tokens (Qwen-Image's text-then-image layout). Generation uses a
torch.Generator seeded per tensor, on the requested device (CPU generation is
the portable one: parity tests generate on the CPU and copy to the GPU).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch


@dataclass(frozen=True)
class Config:
    name: str
    H: int
    S: int
    D: int = 128
    dist: str = "iid"          # "iid" N(0,1) | "rms_gain" RMS-norm x U(0.5,1.5) gain | "rms"
    text: int = 0              # text slots at the front of the sequence
    text_valid: int = 0        # how many text slots are valid keys (seeded choice)
    k_outliers: int = 0        # K channels per head with a constant N(0, var 4) offset


CONFIGS = {
    1: Config("cpu_plumbing_h24_s1088", H=24, S=1088),
    2: Config("qwen_image_1024_h24_s4352", H=24, S=4352, dist="rms_gain", text=256, text_valid=200),
    3: Config("qwen_image_1024_sage_h24_s4352", H=24, S=4352, dist="rms_gain", text=256, text_valid=200,
              k_outliers=8),
    4: Config("qwen_image_edit2_h24_s12544", H=24, S=12544, dist="rms_gain", text=256, text_valid=180),
    5: Config("minimax_h3_video_h40_s32760", H=40, S=32760, dist="rms", k_outliers=8),
}


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _qk(cfg: Config, seed: int, device, k_side: bool) -> torch.Tensor:
    g = _gen(seed, device)
    x = torch.randn(cfg.S, cfg.H, cfg.D, generator=g, device=device, dtype=torch.float32)
    if cfg.dist in ("rms_gain", "rms"):
        x = x * torch.rsqrt(x.square().mean(-1, keepdim=True) + 1e-6)
        if cfg.dist == "rms_gain":
            gain = torch.rand(cfg.D, generator=g, device=device) + 0.5
            x = x * gain
    if k_side and cfg.k_outliers:
        for h in range(cfg.H):
            ch = torch.randperm(cfg.D, generator=g, device=device)[: cfg.k_outliers]
            off = 2.0 * torch.randn(cfg.k_outliers, generator=g, device=device)
            x[:, h, ch] += off
    return x.to(torch.bfloat16)


def make_mask(cfg: Config, seed: int, device="cpu") -> Optional[torch.Tensor]:
    if not cfg.text:
        return None
    g = _gen(seed + 3, "cpu")
    m = torch.ones(cfg.S, dtype=torch.uint8)
    m[: cfg.text] = 0
    m[torch.randperm(cfg.text, generator=g)[: cfg.text_valid]] = 1
    return m.to(device)


def make_inputs(cfg: Config, seed: int = 0, device="cpu"):
    """(q, k, v, kv_valid) for `cfg`: q/k/v [S,H,D] bf16 on `device`, mask uint8 [S] or None."""
    q = _qk(cfg, seed * 10 + 1, device, False)
    k = _qk(cfg, seed * 10 + 2, device, True)
    v = torch.randn(cfg.S, cfg.H, cfg.D, generator=_gen(seed * 10 + 3, device), device=device,
                    dtype=torch.float32).to(torch.bfloat16)
    return q, k, v, make_mask(cfg, seed, device)


def attn_flops(H: int, Sq: int, Skv: int, D: int = 128) -> float:
    """Nominal attention FLOP: 4*H*Sq*Skv*D."""
    return 4.0 * H * Sq * Skv * D

"""MI355X (gfx950) DiT joint self-attention: BF16 flash attention and Sage INT8/FP8
attention, hand-written HIP kernels behind a C ABI (include/miroxen_attn.h)."""
from .attention import (ROPE_HALF, ROPE_INTERLEAVED, ROPE_NONE, AttnParams, attn_reference, flash_attn,
                        flash_attn_fp8, flash_attn_fp8_ok, flash_attn_fp8_supported, flash_attn_fp8_workspace,
                        flash_attn_fp8_norm_rope, head_norm_rope, sage_attend, sage_layout, sage_quantize,
                        sage_quantize_norm_rope, version)

from . import blockscale  # noqa: E402  (block-scaled GEMM: QMode, quantize_blockscaled, gemm_blockscaled)

__all__ = ["blockscale", "AttnParams", "attn_reference", "flash_attn", "flash_attn_fp8", "flash_attn_fp8_ok",
           "flash_attn_fp8_supported", "flash_attn_fp8_workspace", "head_norm_rope", "sage_attend", "sage_layout",
           "sage_quantize", "version", "flash_attn_fp8_norm_rope", "sage_quantize_norm_rope", "ROPE_NONE", "ROPE_INTERLEAVED", "ROPE_HALF"]

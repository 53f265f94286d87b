"""MI355X (gfx950) DiT joint self-attention: BF16 flash attention and Sage INT8/FP8
attention, hand-written HIP kernels behind a C ABI (include/miroxen_attn.h)."""
from .attention import (ROPE_HALF, ROPE_INTERLEAVED, ROPE_NONE, AttnParams, attn_reference, flash_attn,
                        flash_attn_fp8, flash_attn_fp8_ok, flash_attn_fp8_supported, flash_attn_fp8_workspace,
                        head_norm_rope, sage_attend, sage_layout, sage_quantize, version)

__all__ = ["AttnParams", "attn_reference", "flash_attn", "flash_attn_fp8", "flash_attn_fp8_ok",
           "flash_attn_fp8_supported", "flash_attn_fp8_workspace", "head_norm_rope", "sage_attend", "sage_layout",
           "sage_quantize", "version", "ROPE_NONE", "ROPE_INTERLEAVED", "ROPE_HALF"]

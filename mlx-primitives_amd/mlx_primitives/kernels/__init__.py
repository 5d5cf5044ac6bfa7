"""RoPE and fused RoPE + flash attention over the gfx950 kernels."""

from mlx_primitives.kernels.fused_rope_attention import (
    FusedRoPEFlashAttention,
    fast_fused_rope_attention,
    fused_rope_attention,
)
from mlx_primitives.kernels.rope import precompute_rope_cache, rope, rope_at

__all__ = [
    "precompute_rope_cache",
    "rope",
    "rope_at",
    "fused_rope_attention",
    "fast_fused_rope_attention",
    "FusedRoPEFlashAttention",
]

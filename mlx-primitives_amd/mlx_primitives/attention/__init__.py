"""Attention hot path: flash, sliding-window and chunked cross attention.

Same exports as mlx_primitives/attention/__init__.py of the reference for the
functions on this path.
"""

from mlx_primitives.attention.chunked import (
    ChunkedCrossAttention,
    chunked_cross_attention,
    estimate_memory_savings,
)
from mlx_primitives.attention.flash import (
    FlashAttention,
    flash_attention,
    get_optimal_flash_config,
)
from mlx_primitives.attention.sliding_window import (
    SlidingWindowAttention,
    create_sliding_window_mask,
    sliding_window_attention,
)

__all__ = [
    "sliding_window_attention",
    "create_sliding_window_mask",
    "SlidingWindowAttention",
    "flash_attention",
    "FlashAttention",
    "get_optimal_flash_config",
    "chunked_cross_attention",
    "ChunkedCrossAttention",
    "estimate_memory_savings",
]

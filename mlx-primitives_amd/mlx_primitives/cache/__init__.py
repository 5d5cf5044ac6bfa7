"""Paged KV-cache attention (decode and prefill) and page writes over the
reference's page layout."""

from mlx_primitives.cache.kv_store import set_block_data, store_kv
from mlx_primitives.cache.paged_attention import (
    create_block_table_from_lengths,
    get_alibi_slopes,
    paged_attention,
    paged_attention_with_bias,
)

__all__ = [
    "paged_attention",
    "paged_attention_with_bias",
    "create_block_table_from_lengths",
    "get_alibi_slopes",
    "store_kv",
    "set_block_data",
]

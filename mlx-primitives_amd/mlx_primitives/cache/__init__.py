"""Paged KV cache on MI355X: block pools and page tables (host bookkeeping
over device pools), page writes, and paged attention over the reference's page
layout."""

from mlx_primitives.cache.block_allocator import (
    BlockAllocator,
    BlockConfig,
    calculate_num_blocks,
    get_optimal_block_size,
)
from mlx_primitives.cache.kv_cache import (
    CacheMemoryStats,
    KVCache,
    KVCacheConfig,
    MultiLayerKVCache,
)
from mlx_primitives.cache.kv_store import set_block_data, store_kv
from mlx_primitives.cache.page_table import PageTable, SequenceMetadata
from mlx_primitives.cache.paged_attention import (
    create_block_table_from_lengths,
    get_alibi_slopes,
    paged_attention,
    paged_attention_with_bias,
)

__all__ = [
    "BlockAllocator",
    "BlockConfig",
    "CacheMemoryStats",
    "KVCache",
    "KVCacheConfig",
    "MultiLayerKVCache",
    "PageTable",
    "SequenceMetadata",
    "calculate_num_blocks",
    "create_block_table_from_lengths",
    "get_alibi_slopes",
    "get_optimal_block_size",
    "paged_attention",
    "paged_attention_with_bias",
    "set_block_data",
    "store_kv",
]

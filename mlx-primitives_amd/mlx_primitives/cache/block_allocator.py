"""Fixed-size KV-cache blocks in MI355X device memory.

Drop-in for mlx_primitives/cache/block_allocator.py: BlockConfig (18-48),
BlockAllocator (52-379), get_optimal_block_size (382-439) and
calculate_num_blocks (442-452). The K and V pools are torch tensors of shape
(num_blocks, block_size, num_heads, head_dim) on the GPU, the layout the paged
attention kernels read in place; the free list and reference counts are host
bookkeeping. Page writes go through the gfx950 append kernel (store_kv);
copy-on-write duplicates a page with a device-to-device copy.
"""

from __future__ import annotations

import math
import threading
from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch

from mlx_primitives.cache import kv_store

# L2 cache of one MI355X XCD (the cache a workgroup's page reads go through).
MI355X_L2_CACHE_MB = 4.0


def default_device() -> torch.device:
    """The current ROCm device when one is present, else the CPU (pools on the
    CPU hold bookkeeping tests only: page writes and attention need the GPU)."""
    if torch.cuda.is_available():
        return torch.device("cuda", torch.cuda.current_device())
    return torch.device("cpu")


@dataclass(frozen=True)
class BlockConfig:
    """Shape of one KV-cache block (block_allocator.py:18-48).

    block_size: tokens per block; num_heads, head_dim: per-token K (and V)
    rows; dtype: storage type.
    """

    block_size: int = 16
    num_heads: int = 32
    head_dim: int = 128
    dtype: torch.dtype = torch.float16

    @property
    def tokens_per_block(self) -> int:
        return self.block_size

    @property
    def block_bytes(self) -> int:
        """Bytes of one block, K and V together."""
        elem = torch.empty((), dtype=self.dtype).element_size()
        return 2 * self.block_size * self.num_heads * self.head_dim * elem

    @property
    def kv_shape(self) -> Tuple[int, int, int]:
        """(block_size, num_heads, head_dim) of one K or V block."""
        return (self.block_size, self.num_heads, self.head_dim)


class BlockAllocator:
    """Pool of equally sized blocks with O(1) allocate / free and copy-on-write.

    Freed blocks are reused first (last in, first out), so a serving loop
    keeps touching the same pages. Thread-safe (re-entrant lock), as the
    reference (block_allocator.py:52-139).
    """

    def __init__(self, config: BlockConfig, num_blocks: int, enable_cow: bool = True,
                 device=None) -> None:
        self._config = config
        self._num_blocks = num_blocks
        self._enable_cow = enable_cow
        self._lock = threading.RLock()
        self._device = torch.device(device) if device is not None else default_device()
        shape = (num_blocks,) + config.kv_shape
        self._k_pool = torch.zeros(shape, dtype=config.dtype, device=self._device)
        self._v_pool = torch.zeros(shape, dtype=config.dtype, device=self._device)
        # Stack of free ids, lowest on top at start.
        self._free: List[int] = list(range(num_blocks - 1, -1, -1))
        self._ref_counts: List[int] = [0] * num_blocks

    @property
    def config(self) -> BlockConfig:
        return self._config

    @property
    def device(self) -> torch.device:
        return self._device

    @property
    def num_blocks(self) -> int:
        return self._num_blocks

    @property
    def num_free_blocks(self) -> int:
        with self._lock:
            return len(self._free)

    @property
    def num_allocated_blocks(self) -> int:
        with self._lock:
            return self._num_blocks - len(self._free)

    @property
    def memory_usage_bytes(self) -> int:
        return self.num_allocated_blocks * self._config.block_bytes

    @property
    def total_memory_bytes(self) -> int:
        return self._num_blocks * self._config.block_bytes

    def allocate(self, count: int = 1) -> List[int]:
        """Take `count` blocks (reference count 1 each); RuntimeError if the pool
        has fewer free blocks (block_allocator.py:142-167)."""
        with self._lock:
            if count > len(self._free):
                raise RuntimeError(
                    f"Cannot allocate {count} blocks, only {len(self._free)} available")
            out = []
            for _ in range(count):
                block_id = self._free.pop()
                self._ref_counts[block_id] = 1
                out.append(block_id)
            return out

    def _validate_block_id(self, block_id: int, context: str = "") -> None:
        if isinstance(block_id, bool) or not isinstance(block_id, int) or not (
                0 <= block_id < self._num_blocks):
            ctx = f" in {context}" if context else ""
            raise ValueError(f"block_id {block_id} out of bounds [0, {self._num_blocks}){ctx}")

    def free(self, block_ids: List[int]) -> None:
        """Drop one reference to each block; a block returns to the pool when its
        count reaches 0. Blocks that are not allocated are ignored
        (block_allocator.py:185-208)."""
        with self._lock:
            for block_id in block_ids:
                self._validate_block_id(block_id, "free")
                if self._ref_counts[block_id] <= 0:
                    continue
                self._ref_counts[block_id] -= 1
                if self._ref_counts[block_id] == 0:
                    self._free.append(block_id)

    def increment_ref(self, block_id: int) -> None:
        """One more sharer of an allocated block (prefix sharing, forks)."""
        with self._lock:
            self._validate_block_id(block_id, "increment_ref")
            if self._ref_counts[block_id] > 0:
                self._ref_counts[block_id] += 1

    def get_ref_count(self, block_id: int) -> int:
        with self._lock:
            self._validate_block_id(block_id, "get_ref_count")
            return self._ref_counts[block_id]

    def copy_on_write(self, block_id: int) -> int:
        """A block id that is safe to modify: the same block when it has one
        owner (or copy-on-write is off), else a new block holding a device copy
        of its K/V, with the shared block's count decremented
        (block_allocator.py:240-281)."""
        with self._lock:
            self._validate_block_id(block_id, "copy_on_write")
            if not self._enable_cow or self._ref_counts[block_id] <= 1:
                return block_id
            new_id = self.allocate(1)[0]
            self._k_pool[new_id].copy_(self._k_pool[block_id])
            self._v_pool[new_id].copy_(self._v_pool[block_id])
            self._ref_counts[block_id] -= 1
            return new_id

    def get_block_data(self, block_id: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """K and V of one block as views, each (block_size, num_heads, head_dim)."""
        with self._lock:
            self._validate_block_id(block_id, "get_block_data")
            return self._k_pool[block_id], self._v_pool[block_id]

    def set_block_data(self, block_id: int, k: torch.Tensor, v: torch.Tensor, start_pos: int = 0,
                       length: Optional[int] = None) -> int:
        """Write k, v (length, num_heads, head_dim) into slots start_pos.. of a
        block, through copy-on-write when the block is shared
        (block_allocator.py:299-331). Returns the id of the block written (the
        copy when one was made; the reference drops it, so a caller that keeps
        a table must map the old id to this one)."""
        with self._lock:
            self._validate_block_id(block_id, "set_block_data")
            target = self.copy_on_write(block_id) if self._enable_cow else block_id
            kv_store.set_block_data(self._k_pool, self._v_pool, target, k, v, start_pos, length)
            return target

    def get_pools(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """(K_pool, V_pool), each (num_blocks, block_size, num_heads, head_dim)."""
        return self._k_pool, self._v_pool

    def clear(self) -> None:
        """Every block free again (the pool contents are left as they are)."""
        with self._lock:
            self._free = list(range(self._num_blocks - 1, -1, -1))
            self._ref_counts = [0] * self._num_blocks

    def get_stats(self) -> dict:
        with self._lock:
            allocated = self._num_blocks - len(self._free)
            return {
                "num_blocks": self._num_blocks,
                "num_free": len(self._free),
                "num_allocated": allocated,
                "memory_used_mb": allocated * self._config.block_bytes / (1024 * 1024),
                "memory_total_mb": self.total_memory_bytes / (1024 * 1024),
                "utilization": allocated / self._num_blocks if self._num_blocks > 0 else 0.0,
                "cow_enabled": self._enable_cow,
            }


def get_optimal_block_size(head_dim: int, num_heads: int, dtype: torch.dtype = torch.float16,
                           target_l2_fraction: float = 0.5,
                           l2_cache_mb: Optional[float] = None) -> int:
    """Tokens per block so that four K+V blocks fill `target_l2_fraction` of
    the L2 (block_allocator.py:382-439): a power of two in [8, 64]. The L2
    defaults to one MI355X XCD's 4 MB."""
    if l2_cache_mb is None:
        l2_cache_mb = MI355X_L2_CACHE_MB
    elem = torch.empty((), dtype=dtype).element_size()
    kv_per_token = 2 * num_heads * head_dim * elem
    target_bytes = l2_cache_mb * 1024 * 1024 * target_l2_fraction / 4
    block_size = int(target_bytes / kv_per_token)
    block_size = 2 ** int(math.log2(max(8, block_size)))
    return min(max(8, block_size), 64)


def calculate_num_blocks(max_memory_gb: float, config: BlockConfig,
                         reserve_fraction: float = 0.1) -> int:
    """Blocks that fit a memory budget after the reserve
    (block_allocator.py:442-452)."""
    available = max_memory_gb * 1e9 * (1 - reserve_fraction)
    return int(available / config.block_bytes)

"""Paged KV cache for transformer inference on MI355X.

Drop-in for mlx_primitives/cache/kv_cache.py: KVCacheConfig (22-75),
KVCache (78-560) and MultiLayerKVCache (563-640). Per layer a BlockAllocator
holds the K/V pools in device memory and a PageTable maps sequences to their
blocks; `update` appends new tokens with the gfx950 append kernel (positions
and page ids are validated on the host, so an append never waits for the
GPU), and `get_kv_paged` hands the pools, the -1 padded int32 block tables and
the int32 context lengths to `paged_attention` unchanged.

Differences from the reference, each on purpose:
  * a write into a block shared by forked sequences gives the writing
    sequence a private copy and points its table at it (the reference copies
    inside set_block_data but keeps the shared id in the table, so the new
    tokens land in a block no table references);
  * `create_sequence(initial_k, initial_v)` stores the initial tokens (the
    reference reserves the blocks without counting the tokens and then
    raises ValueError for the negative write start);
  * eviction is least-recently-used over whole sequences (`evict_if_needed`);
    the reference's pluggable EvictionPolicy objects are not reproduced, an
    `eviction_policy` passed in only receives its on_create / on_access /
    on_delete notifications.
"""

from __future__ import annotations

import threading
import time
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from mlx_primitives.cache import kv_store
from mlx_primitives.cache.block_allocator import (
    BlockAllocator,
    BlockConfig,
    calculate_num_blocks,
    get_optimal_block_size,
)
from mlx_primitives.cache.page_table import PageTable


@dataclass
class KVCacheConfig:
    """Cache shape and budget (kv_cache.py:22-75). block_size None picks
    get_optimal_block_size for the head shape."""

    num_heads: int
    head_dim: int
    num_layers: int
    max_memory_gb: float = 8.0
    block_size: Optional[int] = None
    dtype: torch.dtype = torch.float16
    enable_cow: bool = True

    def __post_init__(self) -> None:
        if self.block_size is None:
            self.block_size = get_optimal_block_size(self.head_dim, self.num_heads, self.dtype)

    @property
    def block_config(self) -> BlockConfig:
        return BlockConfig(block_size=self.block_size, num_heads=self.num_heads,
                           head_dim=self.head_dim, dtype=self.dtype)

    def calculate_capacity(self) -> Tuple[int, int]:
        """(blocks per layer, max tokens per layer) for the memory budget."""
        blocks = calculate_num_blocks(self.max_memory_gb / self.num_layers, self.block_config)
        return blocks, blocks * self.block_size


@dataclass
class CacheMemoryStats:
    """Memory use of the cache (eviction.py:387-425)."""

    total_bytes: int
    used_bytes: int
    num_sequences: int
    num_blocks_allocated: int
    num_blocks_free: int

    @property
    def utilization(self) -> float:
        return self.used_bytes / self.total_bytes if self.total_bytes > 0 else 0.0

    @property
    def total_mb(self) -> float:
        return self.total_bytes / (1024 * 1024)

    @property
    def used_mb(self) -> float:
        return self.used_bytes / (1024 * 1024)


def _check_rope_positions(rope: Tuple[torch.Tensor, torch.Tensor], end: int) -> None:
    """Positions below `end` must have rows in the RoPE tables."""
    if end > rope[0].shape[0]:
        raise ValueError(f"RoPE position {end - 1} is past the cos/sin tables' "
                         f"{rope[0].shape[0]} rows")


class KVCache:
    """Per-layer paged K/V storage with sequences that grow, fork and shrink."""

    def __init__(self, config: KVCacheConfig, eviction_policy=None, device=None) -> None:
        self._config = config
        self._policy = eviction_policy
        blocks, _ = config.calculate_capacity()
        self._allocators: List[BlockAllocator] = []
        self._page_tables: List[PageTable] = []
        for _ in range(config.num_layers):
            alloc = BlockAllocator(config.block_config, num_blocks=blocks,
                                   enable_cow=config.enable_cow, device=device)
            self._allocators.append(alloc)
            self._page_tables.append(PageTable(alloc))
        # user sequence id -> the sequence id in each layer's page table
        self._sequence_ids: Dict[int, List[int]] = {}
        self._last_access: Dict[int, float] = {}
        self._next_user_seq_id = 0
        self._lock = threading.RLock()

    @property
    def config(self) -> KVCacheConfig:
        return self._config

    @property
    def num_layers(self) -> int:
        return self._config.num_layers

    def _notify(self, event: str, sequence_id: int) -> None:
        self._last_access[sequence_id] = time.monotonic()
        if self._policy is not None and hasattr(self._policy, event):
            getattr(self._policy, event)(sequence_id)

    def _layer_id(self, sequence_id: int, layer_idx: int) -> int:
        if sequence_id not in self._sequence_ids:
            raise KeyError(f"Sequence {sequence_id} not found")
        return self._sequence_ids[sequence_id][layer_idx]

    def create_sequence(self, initial_k: Optional[torch.Tensor] = None,
                        initial_v: Optional[torch.Tensor] = None) -> int:
        """New sequence, with initial (seq_len, heads, dim) K/V stored in every
        layer when given."""
        with self._lock:
            uid = self._next_user_seq_id
            self._next_user_seq_id += 1
            self._sequence_ids[uid] = [pt.create_sequence() for pt in self._page_tables]
            self._notify("on_create", uid)
        if initial_k is not None and initial_v is not None:
            for layer in range(self.num_layers):
                self.update(uid, initial_k, initial_v, layer)
        return uid

    def _store_kv(self, user_seq_id: int, k: torch.Tensor, v: torch.Tensor, layer_idx: int,
                  start_position: Optional[int] = None,
                  rope: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> None:
        """Write k, v (seq_len, heads, dim) at write_start = start_position, or
        num_tokens - seq_len (the tokens extend_sequence just counted), page by
        page through the sequence's table (kv_cache.py:194-264): ValueError for
        a negative start; RuntimeError, after writing the tokens that fit, for a
        position past the table."""
        lsid = self._layer_id(user_seq_id, layer_idx)
        pt = self._page_tables[layer_idx]
        meta = pt.get_sequence_metadata(lsid)
        seq_len = k.shape[0]
        if seq_len == 0:
            return
        write_start = meta.num_tokens - seq_len if start_position is None else start_position
        if write_start < 0:
            raise ValueError(f"Invalid write_start position {write_start}. "
                             f"num_tokens={meta.num_tokens}, seq_len={seq_len}")
        bs = self._config.block_size
        capacity = len(meta.block_table) * bs
        fit = max(0, min(seq_len, capacity - write_start))
        if rope is not None:
            _check_rope_positions(rope, write_start + fit)
        if fit > 0:
            pt.make_writable(lsid, write_start // bs, (write_start + fit - 1) // bs)
            table = pt.get_block_table_tensor([lsid])
            k_pool, v_pool = self._allocators[layer_idx].get_pools()
            kv_store.store_kv(k_pool, v_pool, table, k[:fit][None], v[:fit][None], write_start,
                              check=False, rope=rope)
        if fit < seq_len:
            block_idx = (write_start + fit) // bs
            raise RuntimeError(
                f"Block index {block_idx} out of range. "
                f"Have {len(meta.block_table)} blocks for {meta.num_tokens} tokens.")

    def update(self, sequence_id: int, k: torch.Tensor, v: torch.Tensor, layer_idx: int,
               position: Optional[int] = None, *,
               rope: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> None:
        """Append k, v (new_tokens, heads, dim) to a sequence, or with
        `position` truncate to it first and write there (speculative-decoding
        rollback) (kv_cache.py:266-304).

        rope (keyword-only extension): (cos_cache, sin_cache); K is stored
        rotated to each token's position in the sequence (store_kv)."""
        lsid = self._layer_id(sequence_id, layer_idx)
        self._notify("on_access", sequence_id)
        pt = self._page_tables[layer_idx]
        if rope is not None:
            first = pt.get_sequence_metadata(lsid).num_tokens if position is None else position
            _check_rope_positions(rope, first + k.shape[0])
        if position is None:
            if k.shape[0] == 0:
                return
        else:
            pt.truncate_sequence(lsid, position)
        before = pt.get_sequence_metadata(lsid).num_tokens
        try:
            pt.extend_sequence(lsid, k.shape[0])
            self._store_kv(sequence_id, k, v, layer_idx, rope=rope)
        except Exception:
            # Out of blocks (or a rejected write): the sequence keeps no tokens
            # that no kernel wrote.
            pt.truncate_sequence(lsid, before)
            raise

    def update_batch(self, sequence_ids: Sequence[int], k: torch.Tensor, v: torch.Tensor,
                     layer_idx: int, num_tokens: Optional[Sequence[int]] = None,
                     errors: Optional[torch.Tensor] = None,
                     rope: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> None:
        """Append to several sequences with one kernel launch (a serving step).

        k, v: (batch, T, heads, dim); num_tokens: tokens of each row to append
        (default T, ragged appends otherwise). Equivalent to calling update for
        each sequence in turn; `errors` (int32 (3,), device; (4,) with rope)
        receives the kernel's error words instead of a temporary (they stay
        zero: every position written here was allocated just before, and
        checked against the rope tables). rope: as in update."""
        if k.ndim != 4 or v.shape != k.shape or k.shape[0] != len(sequence_ids):
            raise ValueError(f"k and v must be (len(sequence_ids), T, heads, dim), got "
                             f"{tuple(k.shape)} and {tuple(v.shape)}")
        counts = [k.shape[1]] * len(sequence_ids) if num_tokens is None else list(num_tokens)
        if len(counts) != len(sequence_ids) or any(c < 0 or c > k.shape[1] for c in counts):
            raise ValueError(f"num_tokens must give 0..{k.shape[1]} tokens per sequence")
        if len(set(sequence_ids)) != len(sequence_ids):
            raise ValueError("update_batch: sequence_ids must be distinct (one append per "
                             "sequence and step)")
        pt = self._page_tables[layer_idx]
        bs = self._config.block_size
        if rope is not None:
            _check_rope_positions(rope, max(
                pt.get_sequence_metadata(self._layer_id(sid, layer_idx)).num_tokens + n
                for sid, n in zip(sequence_ids, counts)))
        lsids, starts = [], []
        try:
            for sid, n in zip(sequence_ids, counts):
                lsid = self._layer_id(sid, layer_idx)
                self._notify("on_access", sid)
                start = pt.get_sequence_metadata(lsid).num_tokens
                lsids.append(lsid)
                starts.append(start)
                if n > 0:
                    pt.extend_sequence(lsid, n)
                    pt.make_writable(lsid, start // bs, (start + n - 1) // bs)
        except Exception:
            # The pool ran out partway: every sequence of the batch goes back to
            # its length before the call (blocks allocated here are freed), so
            # none counts tokens that the kernel never wrote.
            for lsid, start in zip(lsids, starts):
                pt.truncate_sequence(lsid, start)
            raise
        if not any(counts):
            return
        tables = pt.get_block_table_tensor(lsids)
        k_pool, v_pool = self._allocators[layer_idx].get_pools()
        dev = k_pool.device
        kv_store.store_kv(k_pool, v_pool, tables, k, v,
                          torch.tensor(starts, dtype=torch.int32).to(dev),
                          torch.tensor(counts, dtype=torch.int32).to(dev), check=False,
                          errors=errors, rope=rope)

    def get_kv(self, sequence_id: int, layer_idx: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """All cached K, V of a sequence, materialized (num_tokens, heads, dim)."""
        lsid = self._layer_id(sequence_id, layer_idx)
        self._notify("on_access", sequence_id)
        meta = self._page_tables[layer_idx].get_sequence_metadata(lsid)
        k_pool, v_pool = self._allocators[layer_idx].get_pools()
        if meta.num_tokens == 0:
            shape = (0, self._config.num_heads, self._config.head_dim)
            return (torch.zeros(shape, dtype=self._config.dtype, device=k_pool.device),
                    torch.zeros(shape, dtype=self._config.dtype, device=k_pool.device))
        idx = torch.tensor(meta.block_table, dtype=torch.long).to(k_pool.device)
        shape = (-1, self._config.num_heads, self._config.head_dim)
        return (k_pool[idx].reshape(shape)[:meta.num_tokens],
                v_pool[idx].reshape(shape)[:meta.num_tokens])

    def get_kv_paged(self, sequence_ids: List[int], layer_idx: int
                     ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        """(K_pool, V_pool, block_tables, context_lens) for paged_attention
        (kv_cache.py:360-394): pools (num_blocks, block_size, heads, dim),
        int32 (batch, max_blocks) tables padded with -1, int32 (batch,)."""
        lsids = [self._layer_id(sid, layer_idx) for sid in sequence_ids]
        for sid in sequence_ids:
            self._notify("on_access", sid)
        pt = self._page_tables[layer_idx]
        k_pool, v_pool = self._allocators[layer_idx].get_pools()
        return k_pool, v_pool, pt.get_block_table_tensor(lsids), pt.get_context_lengths(lsids)

    def fork_sequence(self, sequence_id: int) -> int:
        """New sequence sharing the prefix blocks of `sequence_id` in every layer."""
        with self._lock:
            if sequence_id not in self._sequence_ids:
                raise KeyError(f"Sequence {sequence_id} not found")
            uid = self._next_user_seq_id
            self._next_user_seq_id += 1
            self._sequence_ids[uid] = [pt.fork_sequence(lsid) for pt, lsid in
                                       zip(self._page_tables, self._sequence_ids[sequence_id])]
            self._notify("on_create", uid)
            return uid

    def delete_sequence(self, sequence_id: int) -> None:
        with self._lock:
            if sequence_id not in self._sequence_ids:
                raise KeyError(f"Sequence {sequence_id} not found")
            for pt, lsid in zip(self._page_tables, self._sequence_ids[sequence_id]):
                pt.delete_sequence(lsid)
            del self._sequence_ids[sequence_id]
            self._last_access.pop(sequence_id, None)
            if self._policy is not None and hasattr(self._policy, "on_delete"):
                self._policy.on_delete(sequence_id)

    def get_sequence_length(self, sequence_id: int) -> int:
        lsid = self._layer_id(sequence_id, 0)
        return self._page_tables[0].get_sequence_metadata(lsid).num_tokens

    def clear(self) -> None:
        with self._lock:
            for pt in self._page_tables:
                pt.clear()
            for alloc in self._allocators:
                alloc.clear()
            self._sequence_ids.clear()
            self._last_access.clear()

    @property
    def memory_stats(self) -> CacheMemoryStats:
        return CacheMemoryStats(
            total_bytes=sum(a.total_memory_bytes for a in self._allocators),
            used_bytes=sum(a.memory_usage_bytes for a in self._allocators),
            num_sequences=len(self._sequence_ids),
            num_blocks_allocated=sum(a.num_allocated_blocks for a in self._allocators),
            num_blocks_free=sum(a.num_free_blocks for a in self._allocators))

    def get_all_sequence_ids(self) -> List[int]:
        return list(self._sequence_ids.keys())

    def evict_if_needed(self, bytes_needed: int,
                        protected_sequences: Optional[List[int]] = None) -> int:
        """Delete least-recently-used sequences (not in protected_sequences)
        until `bytes_needed` more bytes fit the cache; returns how many were
        deleted."""
        protected = set(protected_sequences or [])
        evicted = 0
        with self._lock:
            stats = self.memory_stats
            while stats.used_bytes + bytes_needed > stats.total_bytes:
                victims = sorted((t, s) for s, t in self._last_access.items()
                                 if s not in protected and s in self._sequence_ids)
                if not victims:
                    break
                self.delete_sequence(victims[0][1])
                evicted += 1
                stats = self.memory_stats
        return evicted


class MultiLayerKVCache:
    """Convenience wrapper (kv_cache.py:563-640)."""

    def __init__(self, cache: KVCache) -> None:
        self._cache = cache

    @classmethod
    def from_model_config(cls, num_layers: int, num_heads: int, head_dim: int,
                          max_memory_gb: float = 8.0, block_size: Optional[int] = None,
                          dtype: torch.dtype = torch.float16, device=None) -> "MultiLayerKVCache":
        config = KVCacheConfig(num_heads=num_heads, head_dim=head_dim, num_layers=num_layers,
                               max_memory_gb=max_memory_gb, block_size=block_size, dtype=dtype)
        return cls(KVCache(config, device=device))

    def create_sequence(self) -> int:
        return self._cache.create_sequence()

    def get_or_update(self, sequence_id: int, layer_idx: int, new_k: torch.Tensor,
                      new_v: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Append new K/V, then return the sequence's whole K/V."""
        self._cache.update(sequence_id, new_k, new_v, layer_idx)
        return self._cache.get_kv(sequence_id, layer_idx)

    def delete_sequence(self, sequence_id: int) -> None:
        self._cache.delete_sequence(sequence_id)

    def clear(self) -> None:
        self._cache.clear()

    @property
    def inner(self) -> KVCache:
        return self._cache

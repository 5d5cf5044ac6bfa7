"""Page tables of the paged KV cache: logical token positions -> blocks.

Drop-in for mlx_primitives/cache/page_table.py (SequenceMetadata 28-76,
PageTable 79-447). Host bookkeeping per sequence (its block list and token
count) over a BlockAllocator; the batched views the kernels read are built as
int32 device tensors: get_block_table_tensor (B, max_blocks) padded with -1
(295-332) and get_context_lengths (B,) (334-345).
"""

from __future__ import annotations

import threading
import time
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch

from mlx_primitives.cache.block_allocator import BlockAllocator


@dataclass
class SequenceMetadata:
    """One sequence's pages and counts (page_table.py:28-76)."""

    sequence_id: int
    block_table: List[int] = field(default_factory=list)
    num_tokens: int = 0
    num_tokens_in_last_block: int = 0
    last_access_time: float = field(default_factory=time.time)
    ref_count: int = 1
    is_speculative: bool = False
    parent_sequence_id: Optional[int] = None

    def touch(self) -> None:
        self.last_access_time = time.time()


class PageTable:
    """Sequences -> physical blocks, with growth, truncation, forks sharing
    prefix blocks by reference count, and batched tables for paged attention.
    Thread-safe (re-entrant lock)."""

    def __init__(self, block_allocator: BlockAllocator) -> None:
        self._allocator = block_allocator
        self._sequences: Dict[int, SequenceMetadata] = {}
        self._next_sequence_id = 0
        self._lock = threading.RLock()

    @property
    def allocator(self) -> BlockAllocator:
        return self._allocator

    @property
    def num_sequences(self) -> int:
        with self._lock:
            return len(self._sequences)

    @property
    def block_size(self) -> int:
        return self._allocator.config.block_size

    def _get(self, sequence_id: int) -> SequenceMetadata:
        if sequence_id not in self._sequences:
            raise KeyError(f"Sequence {sequence_id} not found")
        return self._sequences[sequence_id]

    def create_sequence(self, initial_tokens: int = 0, parent_sequence_id: Optional[int] = None,
                        is_speculative: bool = False) -> int:
        """New empty sequence; `initial_tokens` reserves blocks for that many
        tokens without counting them as cached (page_table.py:131-165)."""
        with self._lock:
            sid = self._next_sequence_id
            self._next_sequence_id += 1
            self._sequences[sid] = SequenceMetadata(sequence_id=sid, is_speculative=is_speculative,
                                                    parent_sequence_id=parent_sequence_id)
            if initial_tokens > 0:
                self._allocate_blocks_for_tokens(sid, initial_tokens)
            return sid

    def _allocate_blocks_for_tokens(self, sequence_id: int, num_tokens: int) -> None:
        meta = self._sequences[sequence_id]
        needed = (num_tokens + self.block_size - 1) // self.block_size - len(meta.block_table)
        if needed > 0:
            meta.block_table.extend(self._allocator.allocate(needed))

    def _set_count(self, meta: SequenceMetadata, n: int) -> None:
        meta.num_tokens = n
        last = n % self.block_size
        meta.num_tokens_in_last_block = self.block_size if (last == 0 and n > 0) else last

    def extend_sequence(self, sequence_id: int, num_new_tokens: int) -> None:
        """Count `num_new_tokens` more tokens, allocating blocks as needed
        (page_table.py:188-213)."""
        with self._lock:
            meta = self._get(sequence_id)
            meta.touch()
            total = meta.num_tokens + num_new_tokens
            self._allocate_blocks_for_tokens(sequence_id, total)
            self._set_count(meta, total)

    def truncate_sequence(self, sequence_id: int, new_length: int) -> None:
        """Shorten a sequence, freeing the blocks past it (page_table.py:215-245)."""
        with self._lock:
            meta = self._get(sequence_id)
            if new_length >= meta.num_tokens:
                return
            keep = 0 if new_length == 0 else (new_length + self.block_size - 1) // self.block_size
            excess = meta.block_table[keep:]
            if excess:
                self._allocator.free(excess)
                meta.block_table = meta.block_table[:keep]
            self._set_count(meta, new_length)

    def fork_sequence(self, sequence_id: int, is_speculative: bool = False) -> int:
        """New sequence sharing every block of `sequence_id` (each block's count
        goes up by one; writes into a shared block copy it first)."""
        with self._lock:
            parent = self._get(sequence_id)
            nid = self._next_sequence_id
            self._next_sequence_id += 1
            for block_id in parent.block_table:
                self._allocator.increment_ref(block_id)
            self._sequences[nid] = SequenceMetadata(
                sequence_id=nid, block_table=parent.block_table.copy(),
                num_tokens=parent.num_tokens,
                num_tokens_in_last_block=parent.num_tokens_in_last_block,
                is_speculative=is_speculative, parent_sequence_id=sequence_id)
            return nid

    def make_writable(self, sequence_id: int, first_block: int, last_block: int) -> None:
        """Give the sequence private copies of its shared blocks with indices
        first_block..last_block before they are written (copy-on-write at the
        table: the reference copies inside set_block_data but keeps the shared
        id in the table, so the write would land in a block no table
        references)."""
        with self._lock:
            meta = self._get(sequence_id)
            for i in range(max(first_block, 0), min(last_block, len(meta.block_table) - 1) + 1):
                meta.block_table[i] = self._allocator.copy_on_write(meta.block_table[i])

    def get_block_table(self, sequence_id: int) -> List[int]:
        with self._lock:
            meta = self._get(sequence_id)
            meta.touch()
            return meta.block_table.copy()

    def get_block_table_tensor(self, sequence_ids: List[int],
                               max_blocks: Optional[int] = None) -> torch.Tensor:
        """int32 (batch, max_blocks) on the pools' device, -1 padded; longer
        tables are cut to max_blocks (page_table.py:295-332)."""
        dev = self._allocator.device
        with self._lock:
            if not sequence_ids:
                return torch.empty((0,), dtype=torch.int32, device=dev)
            tables = []
            for sid in sequence_ids:
                meta = self._get(sid)
                meta.touch()
                tables.append(meta.block_table.copy())
        if max_blocks is None:
            max_blocks = max(len(t) for t in tables)
        rows = [t[:max_blocks] + [-1] * (max_blocks - len(t[:max_blocks])) for t in tables]
        return torch.tensor(rows, dtype=torch.int32).to(dev, non_blocking=True)

    def get_context_lengths(self, sequence_ids: List[int]) -> torch.Tensor:
        """int32 (batch,) cached tokens per sequence, on the pools' device."""
        with self._lock:
            lengths = [self._get(sid).num_tokens for sid in sequence_ids]
        return torch.tensor(lengths, dtype=torch.int32).to(self._allocator.device,
                                                           non_blocking=True)

    def get_sequence_metadata(self, sequence_id: int) -> SequenceMetadata:
        with self._lock:
            return self._get(sequence_id)

    def get_token_position(self, sequence_id: int, token_idx: int) -> Tuple[int, int]:
        """(block id, slot) of a token (page_table.py:361-374)."""
        with self._lock:
            meta = self._get(sequence_id)
            return meta.block_table[token_idx // self.block_size], token_idx % self.block_size

    def delete_sequence(self, sequence_id: int) -> None:
        """Free a sequence's blocks (shared ones lose one reference)."""
        with self._lock:
            if sequence_id not in self._sequences:
                return
            self._allocator.free(self._sequences[sequence_id].block_table)
            del self._sequences[sequence_id]

    def get_all_sequence_ids(self) -> List[int]:
        with self._lock:
            return list(self._sequences.keys())

    def get_sequences_by_access_time(self, ascending: bool = True) -> List[int]:
        with self._lock:
            return sorted(self._sequences, key=lambda s: self._sequences[s].last_access_time,
                          reverse=not ascending)

    def clear(self) -> None:
        with self._lock:
            for sid in list(self._sequences):
                self.delete_sequence(sid)

    def get_stats(self) -> dict:
        with self._lock:
            tokens = sum(m.num_tokens for m in self._sequences.values())
            blocks = sum(len(m.block_table) for m in self._sequences.values())
            return {
                "num_sequences": len(self._sequences),
                "total_tokens": tokens,
                "total_blocks": blocks,
                "avg_tokens_per_sequence": tokens / len(self._sequences) if self._sequences else 0,
                "avg_blocks_per_sequence": blocks / len(self._sequences) if self._sequences else 0,
            }

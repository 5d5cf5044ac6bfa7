"""CPU oracle: restatement of mlx-primitives' KV-cache page writes in NumPy.

TEST INFRASTRUCTURE ONLY (see oracle/attention.py for the import rule).

Restates KVCache._store_kv (mlx_primitives/cache/kv_cache.py:194-264) and the
BlockAllocator.set_block_data writes it issues
(mlx_primitives/cache/block_allocator.py:299-331) over the pools
(num_blocks, block_size, H, D): the new tokens are written block by block,
each chunk being the run of tokens that fits in the current page.

Parity pins (tests/test_oracle.py): write-then-gather round trips (every
appended token read back through the block table equals the input, every
other slot is unchanged), the reference's set/get known-answer test
(tests/cache/test_block_allocator.py:97-119), and the reference's three error
cases.
"""

from __future__ import annotations

from typing import Optional, Sequence

import numpy as np


def set_block_data(k_pool: np.ndarray, v_pool: np.ndarray, block_id: int, k: np.ndarray,
                   v: np.ndarray, start_pos: int = 0, length: Optional[int] = None) -> None:
    """Write k, v into one page from slot start_pos.

    Restates mlx_primitives/cache/block_allocator.py:299-331 (without
    copy-on-write, which is a bookkeeping concern of the allocator); the
    bounds check is BlockAllocator._validate_block_id's ValueError.
    """
    if block_id < 0 or block_id >= k_pool.shape[0]:
        raise ValueError(f"Invalid block_id {block_id}")
    if length is None:
        length = k.shape[0]
    end = start_pos + length
    k_pool[block_id, start_pos:end] = k
    v_pool[block_id, start_pos:end] = v


def store_kv(k_pool: np.ndarray, v_pool: np.ndarray, block_table: Sequence[int], k: np.ndarray,
             v: np.ndarray, write_start: int, block_size: int) -> None:
    """Write one sequence's new tokens (seq_len, H, D) from position write_start.

    Restates mlx_primitives/cache/kv_cache.py:219-264: a negative start raises
    ValueError (236-241), a block index past the table RuntimeError (250-254);
    chunks written before the failing block stay written.
    """
    seq_len = k.shape[0]
    if write_start < 0:
        raise ValueError(f"Invalid write_start position {write_start}")
    written = 0
    while written < seq_len:
        pos = write_start + written
        bi, off = divmod(pos, block_size)
        if bi >= len(block_table):
            raise RuntimeError(f"Block index {bi} out of range")
        n = min(seq_len - written, block_size - off)
        set_block_data(k_pool, v_pool, int(block_table[bi]), k[written:written + n],
                       v[written:written + n], off)
        written += n


def kv_append(k_pool: np.ndarray, v_pool: np.ndarray, block_tables: np.ndarray, k: np.ndarray,
              v: np.ndarray, start_pos: Sequence[int], n_tokens: Optional[Sequence[int]] = None,
              block_size: Optional[int] = None) -> None:
    """Batched store_kv: sequence b writes k[b, :n_tokens[b]] from start_pos[b].

    k, v: (B, T, H, D); block_tables: (B, max_blocks). Sequences are written in
    order; an error in one stops the loop there, as successive reference calls
    would.
    """
    bsz, T = k.shape[:2]
    if block_size is None:
        block_size = k_pool.shape[1]
    if n_tokens is None:
        n_tokens = [T] * bsz
    for b in range(bsz):
        n = int(n_tokens[b])
        store_kv(k_pool, v_pool, np.asarray(block_tables[b]), k[b, :n], v[b, :n],
                 int(start_pos[b]), block_size)

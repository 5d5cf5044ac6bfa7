"""Writes of new K/V tokens into a paged KV cache on MI355X.

Drop-in for the page writes of the reference's KV cache:
KVCache._store_kv (mlx_primitives/cache/kv_cache.py:194-264) and
BlockAllocator.set_block_data (mlx_primitives/cache/block_allocator.py:299-331),
over the same pools (num_blocks, block_size, H, D) and int32 block tables
padded with -1. One gfx950 scatter kernel writes every new token of every
sequence into its page slot; the allocator bookkeeping (which pages a sequence
owns, eviction, copy-on-write) stays with the caller.
"""

from __future__ import annotations

from typing import Optional, Tuple, Union

import torch

from mlx_primitives import _native


def _i32(x, device, n: int, what: str) -> torch.Tensor:
    t = torch.as_tensor(x, dtype=torch.int32, device=device).reshape(-1)
    if t.numel() == 1 and n > 1:
        t = t.expand(n)
    if t.numel() != n:
        raise ValueError(f"{what} must have {n} entries, got {t.numel()}")
    return t.contiguous()


def _raise_errors(flags) -> None:
    neg, past, bad = (int(x) for x in flags[:3])
    if len(flags) > 3 and int(flags[3]):
        raise ValueError("RoPE position out of range: a token's position lies past the "
                         "cos/sin tables")
    if neg:
        raise ValueError("Invalid write_start position: a start position is negative")
    if past:
        raise RuntimeError("Block index out of range: a token's position lies past its "
                           "sequence's block table")
    if bad:
        raise ValueError("Invalid block_id: a block table entry is outside the pool")


def store_kv(
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    block_tables: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    start_positions: Union[int, torch.Tensor],
    num_tokens: Optional[Union[int, torch.Tensor]] = None,
    check: bool = True,
    errors: Optional[torch.Tensor] = None,
    rope: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
) -> Optional[torch.Tensor]:
    """Write new tokens into their pages, in place.

    k, v: (batch, T, heads, dim), or (T, heads, dim) for one sequence as in
    KVCache._store_kv; block_tables: (batch, max_blocks) or (max_blocks,);
    start_positions: position of each sequence's first new token (int or
    (batch,)); num_tokens: tokens to write per sequence (default T), for
    ragged appends. Token t of sequence b lands at position p = start + t,
    page block_tables[b, p // block_size], slot p % block_size.

    With ``check`` (the default) the call waits for the kernel and raises like
    the reference: ValueError for a negative start, RuntimeError for a
    position past the block table, ValueError for a page id outside the pool.
    Unlike the reference, which stops at the failing chunk, every token that
    can be placed is written. With ``check=False`` nothing waits and the int32
    (3,) error words [negative start, past table, bad page] are returned.

    errors: optional int32 (3,) device tensor that receives the error words
    (cleared by a fill kernel, then set by the append kernel), so that a call
    allocates nothing, e.g. inside a captured HIP graph; without it a
    temporary is allocated per call.

    rope (keyword-only extension): (cos_cache, sin_cache) tables as built by
    precompute_rope_cache, (positions, dim // 2). Each K token is stored
    rotated to its position p (the values rope(k, cos, sin, p) gives, in the
    same kernel that writes the pages), V as given, so attention over the
    cache rotates only its queries. The error words are then 4, the fourth
    set for a position at or past the tables' rows (ValueError with check).
    """
    if k.ndim == 3:
        k, v = k[None], v[None]
        block_tables = block_tables.reshape(1, -1)
    if k.ndim != 4 or v.shape != k.shape:
        raise ValueError(
            f"k and v must both be (batch, T, heads, dim); got {tuple(k.shape)} and "
            f"{tuple(v.shape)}")
    if k_pool.ndim != 4 or v_pool.shape != k_pool.shape:
        raise ValueError(
            f"k_pool and v_pool must both be (num_blocks, block_size, heads, dim); got "
            f"{tuple(k_pool.shape)} and {tuple(v_pool.shape)}")
    batch, T, heads, dim = k.shape
    num_blocks, block_size = k_pool.shape[:2]
    if k_pool.shape[2:] != (heads, dim):
        raise ValueError(f"pool heads/dim {tuple(k_pool.shape[2:])} do not match k ({heads}, {dim})")
    if k.dtype != k_pool.dtype or v.dtype != k_pool.dtype or v_pool.dtype != k_pool.dtype:
        raise ValueError(f"k/v/pool dtype mismatch: {k.dtype}, {v.dtype}, {k_pool.dtype}")
    if block_tables.ndim != 2 or block_tables.shape[0] != batch:
        raise ValueError(f"block_tables must be (batch, max_blocks), got {tuple(block_tables.shape)}")
    if not (k_pool.is_contiguous() and v_pool.is_contiguous()):
        raise ValueError("k_pool and v_pool must be contiguous (they are written in place)")
    dev = _native.require_device(k_pool, v_pool, k, v, block_tables)
    starts = _i32(start_positions, dev, batch, "start_positions")
    counts = _i32(T if num_tokens is None else num_tokens, dev, batch, "num_tokens")
    tables = block_tables if block_tables.dtype == torch.int32 else block_tables.to(torch.int32)
    tables = tables.contiguous()
    es = k.element_size()
    if (dim * es) % 16:
        raise NotImplementedError(
            f"store_kv: head_dim * element size must be a multiple of 16 bytes (dim={dim})")
    vec = 16 // es

    def fit(x: torch.Tensor) -> torch.Tensor:
        if x.stride(-1) != 1 or any(s % vec for s in x.stride()[:3]) or x.data_ptr() % 16:
            return x.contiguous()
        return x
    k, v = fit(k), fit(v)
    n_err = 3 if rope is None else 4
    if rope is not None:
        cos_cache, sin_cache = rope
        if (cos_cache.shape != sin_cache.shape or cos_cache.ndim != 2
                or cos_cache.shape[1] != dim // 2):
            raise ValueError(
                f"rope cos/sin caches must both be (positions, {dim // 2}); got "
                f"{tuple(cos_cache.shape)} and {tuple(sin_cache.shape)}")
        if dim % 16:
            raise NotImplementedError(
                f"store_kv(rope=...): head_dim must be a multiple of 16, got {dim}")
        _native.require_device(cos_cache, sin_cache)
        cos_cache, sin_cache = cos_cache.contiguous(), sin_cache.contiguous()
    if errors is None:
        errors = torch.zeros(n_err, dtype=torch.int32, device=dev)
    else:
        if (errors.dtype != torch.int32 or errors.numel() != n_err or errors.device != dev
                or not errors.is_contiguous()):
            raise ValueError(f"errors must be a contiguous int32 tensor of {n_err} entries on "
                             "the pools' device")
        errors.zero_()
    if rope is None:
        _native.kv_append(k, v, k_pool, v_pool, tables, starts, counts, errors, k.stride()[:3],
                          v.stride()[:3], batch, T, heads, dim, num_blocks, block_size,
                          tables.shape[1])
    else:
        _native.kv_append_rope(k, v, k_pool, v_pool, tables, starts, counts, errors,
                               k.stride()[:3], v.stride()[:3], batch, T, heads, dim, num_blocks,
                               block_size, tables.shape[1], cos_cache, sin_cache)
    if not check:
        return errors
    _raise_errors(errors.tolist())
    return None


def set_block_data(k_pool: torch.Tensor, v_pool: torch.Tensor, block_id: int, k: torch.Tensor,
                   v: torch.Tensor, start_pos: int = 0, length: Optional[int] = None) -> None:
    """Write k, v (length, heads, dim) into page block_id from slot start_pos.

    Same arguments and errors as BlockAllocator.set_block_data
    (block_allocator.py:299-331, without the allocator's copy-on-write).
    """
    num_blocks, block_size = k_pool.shape[:2]
    if not 0 <= int(block_id) < num_blocks:
        raise ValueError(f"Invalid block_id {block_id} (pool has {num_blocks} blocks)")
    if length is None:
        length = k.shape[0]
    if start_pos < 0 or start_pos + length > block_size or length > k.shape[0]:
        raise ValueError(
            f"slots [{start_pos}, {start_pos + length}) do not fit a block of {block_size}")
    table = torch.full((1, 1), int(block_id), dtype=torch.int32, device=k_pool.device)
    store_kv(k_pool, v_pool, table, k[:length][None], v[:length][None], start_pos, check=False)

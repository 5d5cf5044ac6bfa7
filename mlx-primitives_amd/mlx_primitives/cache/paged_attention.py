"""Paged attention on MI355X: the mlx-primitives ``paged_attention`` API.

Drop-in for mlx_primitives/cache/paged_attention.py (get_alibi_slopes 17-41,
paged_attention 44-105, paged_attention_with_bias 323-384,
create_block_table_from_lengths 387-440) over the same KV layout: pools
(num_blocks, block_size, H, D), int32 block tables (B, max_blocks) padded
with -1, int32 context lengths (B,). Decode (seq_q == 1) runs the gfx950
split-K paged-decode kernel and prefill (seq_q > 1) the flash kernel with
block-table indirection; nothing is gathered into a dense tensor.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from mlx_primitives import _native
from mlx_primitives.attention._launch import kernel_head_dim


def get_alibi_slopes(num_heads: int, device=None) -> torch.Tensor:
    """ALiBi slopes ratio**(i+1), ratio = 2**(-8/num_heads), float32 (num_heads,)."""
    ratio = 2.0 ** (-8.0 / num_heads)
    return torch.tensor([ratio ** (i + 1) for i in range(num_heads)], dtype=torch.float32,
                        device=device)


def _as_i32(x: torch.Tensor) -> torch.Tensor:
    if x.dtype != torch.int32:
        x = x.to(torch.int32)
    return x.contiguous()


def paged_attention(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: Optional[float] = None,
    block_size: int = 16,
    causal: bool = True,
    alibi_slopes: Optional[torch.Tensor] = None,
    *,
    enable_gqa: bool = False,
) -> torch.Tensor:
    """Attention of q against a paged KV cache.

    q: (batch, seq_q, heads, dim); k_pool, v_pool: (num_blocks, block_size,
    heads, dim); block_tables: (batch, max_blocks) page ids, -1 = none;
    context_lens: (batch,) cached tokens per sequence; alibi_slopes: optional
    (heads,), bias slope * (kv_pos - q_pos) with q_pos = context_len in decode
    and q_pos = 0..seq_q-1 in prefill.

    Decode (seq_q == 1) ignores ``causal`` like the reference
    (paged_attention.py:108-208). Prefill (seq_q > 1, paged_attention.py:
    211-320) places query i at position i: with ``causal`` it sees cached
    positions <= i. Both run gfx950 kernels that read the pages through the
    block table. Returns (batch, seq_q, heads, dim) in q's dtype. A query row
    with no valid cached token yields NaN (the reference's softmax over an all
    -inf row).

    enable_gqa (keyword-only extension): the pools may carry H_kv heads, heads
    a multiple of H_kv; query head h reads K/V head h // (heads // H_kv).
    """
    if q.ndim != 4:
        raise ValueError(f"Expected q of shape (batch, seq_q, heads, dim), got {q.ndim}D")
    batch, seq_q, heads, dim = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(dim)
    if k_pool.ndim != 4 or v_pool.shape != k_pool.shape:
        raise ValueError(
            f"k_pool and v_pool must both be (num_blocks, block_size, heads, dim); got "
            f"{tuple(k_pool.shape)} and {tuple(v_pool.shape)}")
    if k_pool.shape[1] != block_size:
        raise ValueError(
            f"block_size={block_size} does not match the pool's block dimension "
            f"{k_pool.shape[1]}")
    h_kv = k_pool.shape[2]
    heads_ok = (h_kv > 0 and heads % h_kv == 0) if enable_gqa else h_kv == heads
    if not heads_ok or k_pool.shape[3] != dim:
        raise ValueError(
            f"pool heads/dim {tuple(k_pool.shape[2:])} do not match q ({heads}, {dim})"
            + (" (enable_gqa: pool heads must divide q heads)" if enable_gqa else ""))
    if block_tables.ndim != 2 or block_tables.shape[0] != batch:
        raise ValueError(f"block_tables must be (batch, max_blocks), got {tuple(block_tables.shape)}")
    if context_lens.ndim != 1 or context_lens.shape[0] != batch:
        raise ValueError(f"context_lens must be (batch,), got {tuple(context_lens.shape)}")
    if q.dtype != k_pool.dtype or q.dtype != v_pool.dtype:
        raise ValueError(
            f"q/k_pool/v_pool dtype mismatch: {q.dtype}, {k_pool.dtype}, {v_pool.dtype}")

    _native.require_device(q, k_pool, v_pool, block_tables, context_lens)
    _native.require_no_grad(q, k_pool, v_pool, alibi_slopes)
    if alibi_slopes is not None:
        alibi_slopes = alibi_slopes.to(device=q.device, dtype=torch.float32).contiguous()
        if alibi_slopes.numel() != heads:
            raise ValueError(f"alibi_slopes must have {heads} entries, got {alibi_slopes.numel()}")
    dk = kernel_head_dim(dim, what="paged attention")
    vec = 4 if q.dtype == torch.float32 else 8
    if dk != dim and not (seq_q == 1 and dim % vec == 0):
        # The decode kernel reads pools of any head dim that is a multiple of
        # the 16-byte vector in place. Otherwise only the pages the tables
        # reference are copied, zero-padded to the kernel head dim (exact:
        # zero dims add nothing to q.k); the pools themselves are never copied.
        k_pool, v_pool, block_tables = _referenced_pages_padded(k_pool, v_pool, block_tables, dk)
        q = torch.nn.functional.pad(q, (0, dk - dim))
    else:
        dk = dim
    k_pool = k_pool.contiguous()
    v_pool = v_pool.contiguous()
    if (q.stride(-1) != 1 or q.stride(0) % vec or q.stride(1) % vec or q.stride(2) % vec
            or q.data_ptr() % 16):
        q = q.contiguous()
    tables = _as_i32(block_tables)
    lens = _as_i32(context_lens)
    out = torch.empty((batch, seq_q, heads, dk), dtype=q.dtype, device=q.device)
    if seq_q == 1:
        _native.paged_decode(
            q, k_pool, v_pool, tables, lens, alibi_slopes, out,
            (q.stride(0), q.stride(2)), (out.stride(0), out.stride(2)),
            batch, heads, dk, k_pool.shape[0], block_size, tables.shape[1], scale, H_kv=h_kv)
    else:
        _native.paged_prefill(
            q, k_pool, v_pool, tables, lens, alibi_slopes, out,
            (q.stride(0), q.stride(2), q.stride(1)),
            (out.stride(0), out.stride(2), out.stride(1)),
            batch, seq_q, heads, dk, k_pool.shape[0], block_size, tables.shape[1], scale,
            causal, H_kv=h_kv)
    if dk != dim:
        out = out[..., :dim].contiguous()
    return out


def _referenced_pages_padded(k_pool: torch.Tensor, v_pool: torch.Tensor,
                             block_tables: torch.Tensor, dk: int):
    """Pools holding only the pages block_tables references (ids in range),
    zero-padded to head dim dk, and the tables renumbered to them (-1 kept).
    Moves O(referenced tokens) bytes; reads the number of distinct pages back
    to the host (one synchronisation)."""
    nb = k_pool.shape[0]
    t = block_tables.to(torch.int64)
    valid = (t >= 0) & (t < nb)
    used = torch.unique(t[valid])
    remap = torch.full_like(t, -1)
    remap[valid] = torch.searchsorted(used, t[valid])
    pad = (0, dk - k_pool.shape[-1])
    return (torch.nn.functional.pad(k_pool[used], pad), torch.nn.functional.pad(v_pool[used], pad),
            remap.to(torch.int32))


def paged_attention_with_bias(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    attention_bias: Optional[torch.Tensor] = None,
    alibi_slopes: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    block_size: int = 16,
    causal: bool = True,
) -> torch.Tensor:
    """paged_attention with ALiBi; a general bias is rejected as in the reference
    (paged_attention.py:372-379)."""
    if attention_bias is not None and alibi_slopes is not None:
        raise ValueError("Cannot specify both attention_bias and alibi_slopes")
    if attention_bias is not None:
        raise NotImplementedError(
            "Pre-computed attention_bias support in paged_attention is not yet implemented. "
            "Use alibi_slopes parameter for ALiBi-style position encoding instead.")
    return paged_attention(q, k_pool, v_pool, block_tables, context_lens, scale, block_size,
                           causal, alibi_slopes=alibi_slopes)


def create_block_table_from_lengths(sequence_lengths: torch.Tensor, block_size: int,
                                    max_blocks: Optional[int] = None) -> torch.Tensor:
    """Consecutive page ids per sequence, -1 padded, int32 (batch, max_blocks).

    Same table as mlx_primitives/cache/paged_attention.py:387-440: sequence i
    owns pages [sum of earlier page counts, + ceil(len_i / block_size)).
    """
    lens = sequence_lengths.to(torch.int64)
    per_seq = (lens + block_size - 1) // block_size
    width = int(per_seq.max().item()) if max_blocks is None else int(max_blocks)
    first = torch.cumsum(per_seq, 0) - per_seq
    col = torch.arange(width, device=lens.device)[None, :]
    ids = first[:, None] + col
    return torch.where(col < per_seq[:, None], ids, torch.full_like(ids, -1)).to(torch.int32)

"""CPU oracle: restatement of mlx-primitives' paged attention in NumPy.

TEST INFRASTRUCTURE ONLY (see oracle/attention.py for the import rule).

Restates mlx_primitives/cache/paged_attention.py. The reference's decode path
gathers every page of the block table into a dense (B, max_blocks*bs, H, D)
tensor; this restatement evaluates the same masked softmax one sequence at a
time (same values, bounded memory), so it also runs at the full benchmark size.
"""

from __future__ import annotations

import math
from typing import Optional

import numpy as np


def get_alibi_slopes(num_heads: int) -> np.ndarray:
    """ALiBi slopes ratio**(i+1), ratio = 2**(-8/num_heads).

    Restates mlx_primitives/cache/paged_attention.py:17-41.
    """
    ratio = 2.0 ** (-8.0 / num_heads)
    return np.array([ratio ** (i + 1) for i in range(num_heads)], dtype=np.float32)


def create_block_table_from_lengths(
    sequence_lengths: np.ndarray, block_size: int, max_blocks: Optional[int] = None,
) -> np.ndarray:
    """Sequential page ids per sequence, -1 padded (int32).

    Restates mlx_primitives/cache/paged_attention.py:387-440.
    """
    lens = np.asarray(sequence_lengths, dtype=np.int64)
    per_seq = (lens + block_size - 1) // block_size
    width = int(per_seq.max()) if max_blocks is None else max_blocks
    starts = np.concatenate([[0], np.cumsum(per_seq)[:-1]])
    pos = np.arange(width)[None, :]
    ids = starts[:, None] + pos
    return np.where(pos < per_seq[:, None], ids, -1).astype(np.int32)


def paged_attention_decode(
    q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray, block_tables: np.ndarray,
    context_lens: np.ndarray, scale: float, block_size: int,
    alibi_slopes: Optional[np.ndarray] = None,
) -> np.ndarray:
    """Decode attention over a paged KV cache (q: (B, 1, H, D)).

    Restates mlx_primitives/cache/paged_attention.py:108-208:
      * page ids clamped at 0 for the gather (137), then masked: a position is
        valid iff pos < context_len and its page id >= 0 (184-193);
      * scores = q k^T * scale (+ ALiBi slope_h * (pos - context_len), 163-178);
      * invalid scores = -inf (196); exact softmax (199); output (B, 1, H, D).
    A row with no valid position is NaN (softmax of all -inf), as in the
    reference.
    """
    bsz, _, heads, dim = q.shape
    max_blocks = block_tables.shape[1]
    max_ctx = max_blocks * block_size
    out = np.empty((bsz, 1, heads, v_pool.shape[-1]), dtype=q.dtype)
    pos = np.arange(max_ctx)
    for b in range(bsz):
        tbl = np.asarray(block_tables[b])
        safe = np.maximum(tbl, 0)
        kb = k_pool[safe].reshape(max_ctx, heads, dim)       # gathered pages
        vb = v_pool[safe].reshape(max_ctx, heads, v_pool.shape[-1])
        # (H, T) = per-head k_t . q  (batched matmul over heads)
        scores = np.matmul(np.transpose(kb, (1, 0, 2)), q[b, 0][:, :, None])[..., 0]
        scores = scores * q.dtype.type(scale)
        if alibi_slopes is not None:
            diff = (pos - int(context_lens[b])).astype(np.float32)
            scores = scores + (np.asarray(alibi_slopes, np.float32)[:, None] * diff[None, :]).astype(q.dtype)
        valid = (pos < int(context_lens[b])) & (tbl[pos // block_size] >= 0)
        scores = np.where(valid[None, :], scores, -np.inf)
        with np.errstate(invalid="ignore"):
            m = np.max(scores, axis=-1, keepdims=True)
            e = np.exp(scores - m)
            w = e / np.sum(e, axis=-1, keepdims=True)
        out[b, 0] = np.matmul(w[:, None, :], np.transpose(vb, (1, 0, 2)))[:, 0, :]
    return out


def paged_attention_prefill(
    q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray, block_tables: np.ndarray,
    context_lens: np.ndarray, scale: float, block_size: int, causal: bool,
    alibi_slopes: Optional[np.ndarray] = None,
) -> np.ndarray:
    """Prefill attention over a paged KV cache (q: (B, Sq, H, D)).

    Restates mlx_primitives/cache/paged_attention.py:211-320: validity as in
    decode, ALiBi slope_h * (kv_pos - q_pos) with q_pos = 0..Sq-1, causal
    kv_pos <= q_pos (top-left), exact softmax.
    """
    bsz, seq_q, heads, dim = q.shape
    max_blocks = block_tables.shape[1]
    max_ctx = max_blocks * block_size
    out = np.empty((bsz, seq_q, heads, v_pool.shape[-1]), dtype=q.dtype)
    pos = np.arange(max_ctx)
    qpos = np.arange(seq_q)
    for b in range(bsz):
        tbl = np.asarray(block_tables[b])
        safe = np.maximum(tbl, 0)
        kb = k_pool[safe].reshape(max_ctx, heads, dim)
        vb = v_pool[safe].reshape(max_ctx, heads, v_pool.shape[-1])
        # (H, Sq, T) = per-head q k^T (batched matmul over heads)
        scores = np.matmul(np.transpose(q[b], (1, 0, 2)), np.transpose(kb, (1, 2, 0)))
        scores = scores * q.dtype.type(scale)
        if alibi_slopes is not None:
            diff = (pos[None, :] - qpos[:, None]).astype(np.float32)
            scores = scores + (np.asarray(alibi_slopes, np.float32)[:, None, None] * diff[None]).astype(q.dtype)
        valid = (pos < int(context_lens[b])) & (tbl[pos // block_size] >= 0)
        scores = np.where(valid[None, None, :], scores, -np.inf)
        if causal:
            scores = np.where((pos[None, :] <= qpos[:, None])[None], scores, -np.inf)
        with np.errstate(invalid="ignore"):
            m = np.max(scores, axis=-1, keepdims=True)
            e = np.exp(scores - m)
            w = e / np.sum(e, axis=-1, keepdims=True)
        out[b] = np.transpose(np.matmul(w, np.transpose(vb, (1, 0, 2))), (1, 0, 2))
    return out


def paged_attention(
    q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray, block_tables: np.ndarray,
    context_lens: np.ndarray, scale: Optional[float] = None, block_size: int = 16,
    causal: bool = True, alibi_slopes: Optional[np.ndarray] = None,
) -> np.ndarray:
    """Route on seq_q as mlx_primitives/cache/paged_attention.py:44-105."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if q.shape[1] == 1:
        return paged_attention_decode(q, k_pool, v_pool, block_tables, context_lens, scale,
                                      block_size, alibi_slopes)
    return paged_attention_prefill(q, k_pool, v_pool, block_tables, context_lens, scale,
                                   block_size, causal, alibi_slopes)

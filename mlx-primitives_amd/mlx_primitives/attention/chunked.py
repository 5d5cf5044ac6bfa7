"""Chunked (long-KV) cross-attention on MI355X: the mlx-primitives API.

Drop-in for mlx_primitives/attention/chunked.py (chunked_cross_attention
43-126, ChunkedCrossAttention 410-469, estimate_memory_savings 472-512). The
reference's chunk loop with the online-softmax merge (129-169) becomes split-KV
on the GPU: the KV sequence is divided between workgroups whose (o, m, l)
partials are merged by a second kernel, so memory stays O(Sq * D) whatever
``chunk_size`` is; chunk_size is accepted and only documents the reference's
own chunking.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from mlx_primitives.attention._launch import check_dropout_p, run_attention
from mlx_primitives.constants import Layout


def chunked_cross_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    chunk_size: int = 1024,
    scale: Optional[float] = None,
    causal: bool = False,
    use_metal: bool = True,
    dropout_p: float = 0.0,
    training: bool = True,
) -> torch.Tensor:
    """Cross attention of q (B, Sq, H, D) to long k, v (B, Skv, H, D).

    causal masks kv_pos > q_pos on absolute positions (top-left), as the
    reference (chunked.py:149-154 via compute_chunk_attention). dropout_p > 0
    in training drops attention weights, kept ones scaled by 1 / (1 - dropout_p)
    (chunked.py:109-110, 248-251), with the kernels' counter-based keep mask;
    dropout_p must be in [0, 1).
    """
    if q.ndim != 4:
        raise ValueError(f"Expected 4D tensors (batch, seq, heads, dim), got {q.ndim}D")
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if k.ndim != 4 or v.ndim != 4:
        raise ValueError("k and v must be 4D tensors (batch, seq_kv, heads, dim)")
    if k.shape != v.shape:
        raise ValueError(f"k and v shapes differ: {tuple(k.shape)} vs {tuple(v.shape)}")
    if k.shape[0] != q.shape[0] or k.shape[2] != q.shape[2] or k.shape[3] != q.shape[3]:
        raise ValueError(
            f"q {tuple(q.shape)} and k {tuple(k.shape)} must agree on batch, heads and dim")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError(f"Q/K/V dtype mismatch: Q={q.dtype}, K={k.dtype}, V={v.dtype}")
    drop = dropout_p if training and dropout_p > 0.0 else 0.0
    check_dropout_p(drop, "chunked_cross_attention")
    return run_attention(q, k, v, Layout.BSHD, scale, causal=causal, dropout_p=drop)


class ChunkedCrossAttention:
    """Chunked cross-attention module (chunked.py:410-469), BSHD."""

    def __init__(self, num_heads: int, head_dim: int, chunk_size: int = 1024,
                 causal: bool = False) -> None:
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.chunk_size = chunk_size
        self.causal = causal
        self.scale = 1.0 / math.sqrt(head_dim)

    def __call__(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        return chunked_cross_attention(q, k, v, chunk_size=self.chunk_size,
                                       scale=self.scale, causal=self.causal)


def estimate_memory_savings(seq_q: int, seq_kv: int, num_heads: int, head_dim: int,
                            chunk_size: int, dtype_bytes: int = 4) -> Tuple[int, int, float]:
    """Attention-matrix bytes, dense vs chunked (chunked.py:472-512).

    Returns (dense score bytes, per-chunk score bytes, ratio).
    """
    dense = seq_q * seq_kv * num_heads * dtype_bytes
    chunked = seq_q * chunk_size * num_heads * dtype_bytes
    return dense, chunked, dense / max(chunked, 1)

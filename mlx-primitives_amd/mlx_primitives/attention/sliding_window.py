"""Sliding-window attention on MI355X: the mlx-primitives API.

Drop-in for mlx_primitives/attention/sliding_window.py
(sliding_window_attention 227-313, create_sliding_window_mask 628-656,
SlidingWindowAttention 659-712). The window is the reference's production
convention |i - j| <= window_size (window_size + 1 keys including self), plus
j <= i when causal (sliding_window.py:151-157, 482-491). The gfx950 kernel
applies it by index arithmetic and only visits KV tiles that intersect the
window, so no (S, S) mask is ever built.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from mlx_primitives.attention._launch import check_dropout_p, run_attention
from mlx_primitives.constants import Layout


def sliding_window_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    window_size: int,
    scale: Optional[float] = None,
    causal: bool = True,
    use_metal: bool = True,
    dropout_p: float = 0.0,
    training: bool = True,
) -> torch.Tensor:
    """Attention of each query to keys within window_size positions.

    q, k, v: (batch, seq, heads, dim) ROCm tensors of one dtype.
    window_size: one-sided window; query i sees keys [i - W, i] if causal,
      else [i - W, i + W].
    scale defaults to 1/sqrt(dim); use_metal is accepted and has no effect.
    dropout_p > 0 in training drops attention weights, kept ones scaled by
    1 / (1 - dropout_p) (sliding_window.py:280-282, 617-620), with the kernels'
    counter-based keep mask; dropout_p must be in [0, 1).
    """
    if q.ndim != 4:
        raise ValueError(f"Expected 4D tensors (batch, seq, heads, dim), got {q.ndim}D")
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if window_size < 0:
        raise ValueError(f"window_size must be non-negative, got {window_size}")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(
            f"q, k and v must have the same shape, got {tuple(q.shape)}, {tuple(k.shape)}, "
            f"{tuple(v.shape)}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError(f"Q/K/V dtype mismatch: Q={q.dtype}, K={k.dtype}, V={v.dtype}")
    drop = dropout_p if training and dropout_p > 0.0 else 0.0
    check_dropout_p(drop, "sliding_window_attention")
    window_right = -1 if causal else window_size
    return run_attention(q, k, v, Layout.BSHD, scale, causal=causal,
                         window_left=window_size, window_right=window_right, dropout_p=drop)


def create_sliding_window_mask(seq_len: int, window_size: int, causal: bool = True,
                               device=None) -> torch.Tensor:
    """Boolean (seq_len, seq_len) mask, True where query i may attend key j.

    Same pattern as mlx_primitives/attention/sliding_window.py:628-656.
    """
    pos = torch.arange(seq_len, device=device)
    mask = (pos[:, None] - pos[None, :]).abs() <= window_size
    if causal:
        mask &= pos[None, :] <= pos[:, None]
    return mask


class SlidingWindowAttention:
    """Sliding-window attention module (sliding_window.py:659-712), BSHD."""

    def __init__(self, num_heads: int, head_dim: int, window_size: int,
                 causal: bool = True) -> None:
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.window_size = window_size
        self.causal = causal
        self.scale = 1.0 / math.sqrt(head_dim)

    def __call__(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        return sliding_window_attention(q, k, v, window_size=self.window_size,
                                        scale=self.scale, causal=self.causal)

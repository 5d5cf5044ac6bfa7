"""CPU oracle: restatement of mlx-primitives' RoPE and fused RoPE attention.

TEST INFRASTRUCTURE ONLY (see oracle/attention.py for the import rule).

Restates mlx_primitives/kernels/rope.py (precompute_rope_cache 223-255, the
half-split rotation of rope 476-497) and the fused attention of
kernels/fused_rope_attention.py: rotate Q at positions q_offset + i and K at
kv_offset + j (711-714), then exact softmax attention with the position-based
causal rule of the reference's fused kernel (125-131: key j is visible to
query i when kv_offset + j <= q_offset + i). fast_fused_rope_attention
(637-733) instead hands the rotated tensors to SDPA (716-727), whose causal
rule ignores the offsets (oracle.attention.sdpa_causal_keep).

Parity pins (tests/test_oracle.py): rotation at position 0 is the identity;
rotations preserve each (i, i + D/2) pair's norm; rope(q, m) . rope(k, n)
depends only on m - n (the defining property of RoPE); brute-force loops on
tiny inputs; torch SDPA on the rotated tensors.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np


def precompute_rope_cache(seq_len: int, head_dim: int, base: float = 10000.0,
                          dtype=np.float32) -> Tuple[np.ndarray, np.ndarray]:
    """(seq_len, head_dim // 2) cos/sin of t * base**(-i / (head_dim / 2)), float32
    then cast (rope.py:240-255)."""
    half = head_dim // 2
    inv_freq = np.power(np.float32(base), -np.arange(half, dtype=np.float32) / np.float32(half))
    t = np.arange(seq_len, dtype=np.float32)
    freqs = np.outer(t, inv_freq).astype(np.float32)
    return np.cos(freqs).astype(dtype), np.sin(freqs).astype(dtype)


def rope(x: np.ndarray, cos_cache: np.ndarray, sin_cache: np.ndarray,
         offset: int = 0) -> np.ndarray:
    """Half-split rotation of x (B, S, H, D) at positions offset .. offset+S-1
    (rope.py:477-497), in x's dtype."""
    seq, dim = x.shape[1], x.shape[-1]
    half = dim // 2
    cos = cos_cache[offset:offset + seq][None, :, None, :].astype(x.dtype)
    sin = sin_cache[offset:offset + seq][None, :, None, :].astype(x.dtype)
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * cos - x2 * sin, x1 * sin + x2 * cos], axis=-1)


def fused_rope_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray,
                         scale: Optional[float] = None,
                         cos_cache: Optional[np.ndarray] = None,
                         sin_cache: Optional[np.ndarray] = None, rope_base: float = 10000.0,
                         q_offset: int = 0, kv_offset: int = 0,
                         causal: bool = False) -> np.ndarray:
    """rope(Q), rope(K), then softmax(scale * Q K^T + position-causal mask) V
    (fused_rope_attention.py:637-733 with the mask of 125-131); (B, Sq, H, D).
    A query placed before every key (kv_offset > q_offset + i) sees none and
    gets zeros, as the reference kernel writes them (its running sum stays 0,
    fused_rope_attention.py:176-186)."""
    bsz, seq_q, heads, dim = q.shape
    seq_kv = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(dim)
    if cos_cache is None or sin_cache is None:
        cos_cache, sin_cache = precompute_rope_cache(
            max(seq_q + q_offset, seq_kv + kv_offset), dim, rope_base)
    qr = rope(q, cos_cache, sin_cache, q_offset)
    kr = rope(k, cos_cache, sin_cache, kv_offset)
    # (B, H, Sq, Skv) scores through batched matmul
    s = np.matmul(np.transpose(qr, (0, 2, 1, 3)), np.transpose(kr, (0, 2, 3, 1))) * q.dtype.type(scale)
    if causal:
        qpos = q_offset + np.arange(seq_q)[:, None]
        kpos = kv_offset + np.arange(seq_kv)[None, :]
        s = np.where((kpos <= qpos)[None, None], s, -np.inf)
    with np.errstate(invalid="ignore"):
        m = np.max(s, axis=-1, keepdims=True)
        e = np.exp(s - m)
        w = e / np.sum(e, axis=-1, keepdims=True)
    w = np.where(np.isfinite(m), w, 0.0)  # rows without a visible key
    return np.transpose(np.matmul(w, np.transpose(v, (0, 2, 1, 3))), (0, 2, 1, 3))


def fast_fused_rope_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray,
                              scale: Optional[float] = None,
                              cos_cache: Optional[np.ndarray] = None,
                              sin_cache: Optional[np.ndarray] = None,
                              rope_base: float = 10000.0, q_offset: int = 0,
                              kv_offset: int = 0, causal: bool = False) -> np.ndarray:
    """rope(Q), rope(K) (fused_rope_attention.py:703-714), then SDPA with
    mask="causal" (716-727): the offsets move the rotation only; the causal
    diagonal is SDPA's (key j visible to query i iff j <= i + max(0, Skv - Sq)).
    (B, Sq, H, D)."""
    from oracle.attention import sdpa_attention

    seq_q, dim = q.shape[1], q.shape[-1]
    seq_kv = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(dim)
    if cos_cache is None or sin_cache is None:
        cos_cache, sin_cache = precompute_rope_cache(
            max(seq_q + q_offset, seq_kv + kv_offset), dim, rope_base)
    t = lambda x: np.ascontiguousarray(np.transpose(x, (0, 2, 1, 3)))
    qr = rope(q, cos_cache, sin_cache, q_offset)
    kr = rope(k, cos_cache, sin_cache, kv_offset)
    return np.transpose(sdpa_attention(t(qr), t(kr), t(v), scale, causal), (0, 2, 1, 3))

"""CPU oracle: gradients of mlx-primitives' flash attention, in NumPy.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker; the product
path (mlx_primitives) never calls it.

The reference has no hand-written backward: its tests differentiate
flash_attention, sliding_window_attention and chunked_cross_attention with
mx.grad through the tiled online-softmax path (mlx_primitives/attention/
flash.py:257-316; tests/attention/test_flash.py:338-362,
tests/attention/test_chunked.py:318-339) and compare with PyTorch's
scaled_dot_product_attention backward at ten times the forward tolerance
(tests/parity/pytorch/test_attention_parity.py:107-163, 339-384;
tests/parity/shared/tolerance_config.py:363-387). This module states those
gradients in closed form for the forward O = (E V) / (rowsum E + eps),
E = exp(S - rowmax S) on the kept entries, S = scale * Q K^T:
    P = E / (rowsum E + eps),  dV = P^T dO,  dP = dO V^T,
    dS = P * (dP - rowsum(dO * O)),  dQ = scale * dS K,  dK = scale * dS^T Q
(the eps term and the row max change the result by O(eps) relative only).

Parity pins (tests/test_oracle.py): torch autograd in float64 through the
same forward; torch's scaled_dot_product_attention backward (the routine the
reference's parity suite compares with); central finite differences of
oracle.attention's forward on a tiny case; GQA against autograd through
repeat_interleave of the K/V heads.
"""

from __future__ import annotations

from typing import Tuple

import numpy as np

from oracle.attention import SOFTMAX_EPSILON


def _keep_mask(Sq: int, Sk: int, causal: bool, window_left: int, window_right: int) -> np.ndarray:
    """Kept (query, key) pairs: kv <= q (causal), q - kv <= window_left and
    kv - q <= window_right (sliding_window.py:151-157 window, flash.py causal)."""
    q = np.arange(Sq)[:, None]
    kv = np.arange(Sk)[None, :]
    keep = np.ones((Sq, Sk), dtype=bool)
    if causal:
        keep &= kv <= q
    if window_left >= 0:
        keep &= (q - kv) <= window_left
    if window_right >= 0 and not causal:
        keep &= (kv - q) <= window_right
    return keep


def attention_fwd_bhsd(q, k, v, scale, causal, window_left=-1, window_right=-1,
                       eps=SOFTMAX_EPSILON):
    """(O, P) of the forward above; q (B, H, Sq, D), k/v (B, H_kv, Sk, D) with
    query head h reading K/V head h // (H / H_kv)."""
    g = q.shape[1] // k.shape[1]
    ke, ve = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)
    keep = _keep_mask(q.shape[2], k.shape[2], causal, window_left, window_right)
    s = np.where(keep, scale * (q @ np.swapaxes(ke, -1, -2)), -np.inf)
    m = np.max(s, axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    e = np.where(keep, np.exp(s - m), 0.0)
    p = e / (np.sum(e, axis=-1, keepdims=True) + eps)
    return p @ ve, p


def _score_grad(p: np.ndarray, dp: np.ndarray, dout: np.ndarray, o: np.ndarray) -> np.ndarray:
    """dS = P * (dP - rowsum(dO * O)): the softmax Jacobian applied to dP."""
    return p * (dp - np.sum(dout * o, axis=-1, keepdims=True))


def attention_grad(q: np.ndarray, k: np.ndarray, v: np.ndarray, dout: np.ndarray, scale: float,
                   causal: bool, window_left: int = -1, window_right: int = -1,
                   layout: str = "BSHD", eps: float = SOFTMAX_EPSILON
                   ) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(dq, dk, dv) of sum(out * dout), out = the flash attention forward.

    Tensors are (B, S, H, D) for layout "BSHD", (B, H, S, D) for "BHSD"; K/V
    may carry fewer heads (grouped-query: a K/V head's gradient sums over its
    group of query heads).
    """
    if layout == "BSHD":
        q, k, v, dout = (np.swapaxes(x, 1, 2) for x in (q, k, v, dout))
    B, H, Sq, D = q.shape
    H_kv, Sk = k.shape[1], k.shape[2]
    g = H // H_kv
    ke, ve = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)
    o, p = attention_fwd_bhsd(q, k, v, scale, causal, window_left, window_right, eps)
    dv = np.swapaxes(p, -1, -2) @ dout
    dp = dout @ np.swapaxes(ve, -1, -2)
    ds = _score_grad(p, dp, dout, o)
    dq = scale * (ds @ ke)
    dk = scale * (np.swapaxes(ds, -1, -2) @ q)
    dk = dk.reshape(B, H_kv, g, Sk, D).sum(axis=2)
    dv = dv.reshape(B, H_kv, g, Sk, D).sum(axis=2)
    if layout == "BSHD":
        dq, dk, dv = (np.swapaxes(x, 1, 2) for x in (dq, dk, dv))
    return dq, dk, dv

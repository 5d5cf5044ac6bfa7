"""CPU oracle: attention with dropout on the weights, as the MI355X kernels
compute it, in NumPy.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker; the product
path (mlx_primitives) never calls it.

The reference's training path with dropout_p > 0 (mlx_primitives/attention/
flash.py:202-205 -> 528-578; sliding_window.py:280-282 -> 564-625;
chunked.py:109-110 -> 206-255) computes
    weights = softmax(scores) * keep / (1 - dropout_p),  out = weights @ v,
keep ~ Bernoulli(1 - dropout_p) drawn from MLX's random stream
(mx.random.bernoulli, flash.py:572), which is not reproducible outside MLX.
The kernels replace that draw with a counter-based hash of (seed, row, key),
restated here (the kernels' device code holds the same steps):
    row r = (b * H + h) * Sq + q  (mod 2^32),  key pair m = key // 2,
    bits = lowbias32((r * 0x9E3779B1 + seed_lo) ^ (m * 0x85EBCA77 + seed_hi)),
    key 2m kept iff (bits & 0xffff) >= t,  key 2m + 1 kept iff (bits >> 16) >= t,
    t = min(round(p * 65536), 65535),
lowbias32 being C. Wellons' integer hash (hash-prospector, 2018):
    x ^= x >> 16; x *= 0x7feb352d; x ^= x >> 15; x *= 0x846ca68b; x ^= x >> 16.

Parity pins (tests/test_oracle_dropout.py): lowbias32 against its published inverse
(lowbias32_r: x ^= x >> 16; x *= 0x43021123; x ^= x >> 15 ^ x >> 30;
x *= 0x1d69e2a5; x ^= x >> 16), which undoes it only if every shift and
multiplier matches; the keep mask's statistics (keep rate within 5 sigma of
1 - t / 65536 for both halves of the hash, no correlation between
neighbouring keys, rows or seeds); the forward and gradients against torch
autograd in float64 through the reference's formula with the same mask, and
against oracle.attention_grad when nothing is dropped.
"""

from __future__ import annotations

from typing import Tuple

import numpy as np

from oracle.attention import SOFTMAX_EPSILON
from oracle.attention_grad import _keep_mask as _visible_mask

_G_ROW = np.uint32(0x9E3779B1)
_G_PAIR = np.uint32(0x85EBCA77)


def lowbias32(x: np.ndarray) -> np.ndarray:
    """C. Wellons' lowbias32 on uint32 arrays (wrapping arithmetic)."""
    x = np.asarray(x, dtype=np.uint32).copy()
    with np.errstate(over="ignore"):
        x ^= x >> np.uint32(16)
        x *= np.uint32(0x7FEB352D)
        x ^= x >> np.uint32(15)
        x *= np.uint32(0x846CA68B)
        x ^= x >> np.uint32(16)
    return x


def lowbias32_inverse(x: np.ndarray) -> np.ndarray:
    """The published inverse of lowbias32 (hash-prospector's lowbias32_r)."""
    x = np.asarray(x, dtype=np.uint32).copy()
    with np.errstate(over="ignore"):
        x ^= x >> np.uint32(16)
        x *= np.uint32(0x43021123)
        x ^= (x >> np.uint32(15)) ^ (x >> np.uint32(30))
        x *= np.uint32(0x1D69E2A5)
        x ^= x >> np.uint32(16)
    return x


def threshold(p: float) -> int:
    """Keep threshold of the 16-bit hash halves: round(p * 65536), at most 65535."""
    return min(int(np.floor(p * 65536.0 + 0.5)), 65535)


def keep_mask(B: int, H: int, Sq: int, Sk: int, p: float, seed: int) -> np.ndarray:
    """(B, H, Sq, Sk) bool: True where the kernels keep the weight."""
    return keep_mask_rows(0, B * H * Sq, Sk, p, seed).reshape(B, H, Sq, Sk)


def keep_mask_rows(first_row: int, n_rows: int, Sk: int, p: float, seed: int) -> np.ndarray:
    """(n_rows, Sk) bool keep mask of rows first_row .. first_row + n_rows - 1,
    row r = (b * H + h) * Sq + q as above (one (b, h) slice of a large problem
    without the whole mask)."""
    seed_lo = np.uint32(seed & 0xFFFFFFFF)
    seed_hi = np.uint32((seed >> 32) & 0xFFFFFFFF)
    rows = ((np.arange(n_rows, dtype=np.uint64) + np.uint64(first_row)) &
            np.uint64(0xFFFFFFFF)).astype(np.uint32)
    pairs = np.arange((Sk + 1) // 2, dtype=np.uint32)
    with np.errstate(over="ignore"):
        rk = rows * _G_ROW + seed_lo
        pk = pairs * _G_PAIR + seed_hi
    bits = lowbias32(rk[:, None] ^ pk[None, :])
    t = np.uint32(threshold(p))
    lo = (bits & np.uint32(0xFFFF)) >= t
    hi = (bits >> np.uint32(16)) >= t
    keep = np.empty((n_rows, 2 * pairs.size), dtype=bool)
    keep[:, 0::2] = lo
    keep[:, 1::2] = hi
    return keep[:, :Sk]


def attention_dropout_fwd_bhsd(q, k, v, scale, causal, keep, p, window_left=-1,
                               window_right=-1, eps=SOFTMAX_EPSILON):
    """(O, P) with O = (P * keep / (1 - p)) @ V, P the row softmax of the
    visible scores normalised by (rowsum + eps) like the kernels; q (B, H, Sq,
    D), k / v (B, H_kv, Sk, D), query head h reading K/V head h // (H / H_kv);
    keep (B, H, Sq, Sk)."""
    g = q.shape[1] // k.shape[1]
    ke, ve = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)
    vis = _visible_mask(q.shape[2], k.shape[2], causal, window_left, window_right)
    s = np.where(vis, scale * (q @ np.swapaxes(ke, -1, -2)), -np.inf)
    m = np.max(s, axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    e = np.where(vis, np.exp(s - m), 0.0)
    pr = e / (np.sum(e, axis=-1, keepdims=True) + eps)
    return (pr * keep / (1.0 - p)) @ ve, pr


def attention_dropout(q, k, v, scale, causal, p, seed, window_left=-1, window_right=-1,
                      layout="BSHD"):
    """Forward output of the kernels' dropout attention for (p, seed)."""
    if layout == "BSHD":
        q, k, v = (np.swapaxes(x, 1, 2) for x in (q, k, v))
    B, H, Sq, _ = q.shape
    keep = keep_mask(B, H, Sq, k.shape[2], p, seed)
    o, _ = attention_dropout_fwd_bhsd(q, k, v, scale, causal, keep, p, window_left,
                                      window_right)
    return np.swapaxes(o, 1, 2) if layout == "BSHD" else o


def attention_dropout_grad(q, k, v, dout, scale, causal, p, seed=None, window_left=-1,
                           window_right=-1, layout="BSHD", keep=None, eps=SOFTMAX_EPSILON
                           ) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(dq, dk, dv) of sum(out * dout) for the dropout forward above:
        W = P * keep / (1 - p),  dV = W^T dO,  dW = dO V^T,
        dP = dW * keep / (1 - p),  dS = P * (dP - rowsum(dO * O)),
        dQ = scale * dS K,  dK = scale * dS^T Q,
    rowsum(dP * P) = rowsum(dO * O) because O = W V (exact for eps = 0; the
    kernels' normaliser eps moves it by O(eps) relative). keep defaults to
    keep_mask(..., p, seed)."""
    if layout == "BSHD":
        q, k, v, dout = (np.swapaxes(x, 1, 2) for x in (q, k, v, dout))
    B, H, Sq, D = q.shape
    H_kv, Sk = k.shape[1], k.shape[2]
    g = H // H_kv
    if keep is None:
        keep = keep_mask(B, H, Sq, Sk, p, seed)
    ke, ve = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)
    o, pr = attention_dropout_fwd_bhsd(q, k, v, scale, causal, keep, p, window_left,
                                       window_right, eps)
    w = pr * keep / (1.0 - p)
    dv = np.swapaxes(w, -1, -2) @ dout
    dp = (dout @ np.swapaxes(ve, -1, -2)) * keep / (1.0 - p)
    ds = pr * (dp - np.sum(dout * o, axis=-1, keepdims=True))
    dq = scale * (ds @ ke)
    dk = scale * (np.swapaxes(ds, -1, -2) @ q)
    dk = dk.reshape(B, H_kv, g, Sk, D).sum(axis=2)
    dv = dv.reshape(B, H_kv, g, Sk, D).sum(axis=2)
    if layout == "BSHD":
        dq, dk, dv = (np.swapaxes(x, 1, 2) for x in (dq, dk, dv))
    return dq, dk, dv

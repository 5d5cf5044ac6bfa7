"""CPU oracle: restatement of mlx-primitives' attention algorithms in NumPy.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker (or the timed
CPU baseline); the product path (mlx_primitives) never calls it.

Every function restates one reference function of /root/reference (cited as
file:line) with the same loop structure, block sizes, mask value (-1e38) and
normaliser epsilon (1e-6), so that the oracle reproduces the reference's CPU
fallback path (``use_metal=False``). Arrays are NumPy; computation happens in
the dtype of the inputs (pass float64 for a high-precision oracle, float32 to
mirror the reference's MLX float32 arithmetic).

Parity pins (tests/test_oracle.py): every function here is checked against the
reference tests' known-answer cases, against an independent brute-force loop
evaluation on tiny inputs, against torch.nn.functional.scaled_dot_product_attention
(the library routine the reference's own parity suite compares with), and
against invariants (block/chunk-size independence, merge associativity, full
window == causal).
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np

# mlx_primitives/constants.py:100
ATTENTION_MASK_VALUE = -1e38
# mlx_primitives/constants.py:110
SOFTMAX_EPSILON = 1e-6
# mlx_primitives/constants.py:162-169
FLASH_MAX_SEQ_FOR_REFERENCE = 256
FLASH_SMALL_BATCH_SEQ_THRESHOLD = 512
FLASH_SMALL_BATCH_THRESHOLD = 4


def _bhqk(q: np.ndarray, k: np.ndarray) -> np.ndarray:
    """einsum('bqhd,bkhd->bqhk') through batched matmul (BLAS)."""
    qt = np.transpose(q, (0, 2, 1, 3))  # b h q d
    kt = np.transpose(k, (0, 2, 3, 1))  # b h d k
    return np.transpose(np.matmul(qt, kt), (0, 2, 1, 3))  # b q h k


def _bqhd(p: np.ndarray, v: np.ndarray) -> np.ndarray:
    """einsum('bqhk,bkhd->bqhd') through batched matmul (BLAS)."""
    pt = np.transpose(p, (0, 2, 1, 3))  # b h q k
    vt = np.transpose(v, (0, 2, 1, 3))  # b h k d
    return np.transpose(np.matmul(pt, vt), (0, 2, 1, 3))  # b q h d


def online_softmax_merge(
    acc_output: np.ndarray,
    acc_max: np.ndarray,
    acc_sum: np.ndarray,
    new_output: np.ndarray,
    new_max: np.ndarray,
    new_sum: np.ndarray,
) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Merge two unnormalised (o, m, l) accumulators.

    Restates mlx_primitives/attention/_online_softmax.py:42-106.
    """
    global_max = np.maximum(acc_max, new_max)
    acc_corr = np.exp(acc_max - global_max)
    new_corr = np.exp(new_max - global_max)
    total = acc_sum * acc_corr + new_sum * new_corr
    out = acc_output * acc_corr[..., None] + new_output * new_corr[..., None]
    return out, global_max, total


def compute_chunk_attention(
    q: np.ndarray,
    k_chunk: np.ndarray,
    v_chunk: np.ndarray,
    scale: float,
    causal: bool = False,
    q_offset: int = 0,
    kv_offset: int = 0,
) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Unnormalised attention of q (B, Sq, H, D) against one KV chunk.

    Restates mlx_primitives/attention/_online_softmax.py:109-176: masked scores
    take the finite value -1e38, the chunk max and the exp-sum are per row.
    """
    seq_q = q.shape[1]
    chunk = k_chunk.shape[1]
    scores = _bhqk(q, k_chunk) * q.dtype.type(scale)
    if causal:
        q_pos = np.arange(seq_q) + q_offset
        kv_pos = np.arange(chunk) + kv_offset
        keep = kv_pos[None, :] <= q_pos[:, None]
        scores = np.where(keep[None, :, None, :], scores, q.dtype.type(ATTENTION_MASK_VALUE))
    chunk_max = np.max(scores, axis=-1)
    e = np.exp(scores - chunk_max[..., None])
    chunk_sum = np.sum(e, axis=-1)
    chunk_out = _bqhd(e, v_chunk)
    return chunk_out, chunk_max, chunk_sum


def tiled_flash_attention(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    scale: float,
    causal: bool,
    block_q: int = 32,
    block_kv: int = 32,
) -> np.ndarray:
    """BSHD tiled online-softmax flash attention.

    Restates mlx_primitives/attention/flash.py:257-316: q blocks of block_q,
    kv blocks of block_kv up to q_end (causal) or seq_len (non-causal; the
    reference iterates the *query* length there), o / (l + 1e-6) per q block.
    """
    bsz, seq_len, heads, dim = q.shape
    dt = q.dtype.type
    blocks = []
    for q_start in range(0, seq_len, block_q):
        q_end = min(q_start + block_q, seq_len)
        qb = q[:, q_start:q_end]
        nq = q_end - q_start
        m_i = np.full((bsz, nq, heads), ATTENTION_MASK_VALUE, dtype=q.dtype)
        l_i = np.zeros((bsz, nq, heads), dtype=q.dtype)
        o_i = np.zeros((bsz, nq, heads, dim), dtype=q.dtype)
        kv_limit = q_end if causal else seq_len
        for kv_start in range(0, kv_limit, block_kv):
            kv_end = min(kv_start + block_kv, kv_limit)
            co, cm, cl = compute_chunk_attention(
                qb, k[:, kv_start:kv_end], v[:, kv_start:kv_end], scale,
                causal=causal, q_offset=q_start, kv_offset=kv_start,
            )
            o_i, m_i, l_i = online_softmax_merge(o_i, m_i, l_i, co, cm, cl)
        blocks.append(o_i / (l_i[..., None] + dt(SOFTMAX_EPSILON)))
    return np.concatenate(blocks, axis=1)


def causal_additive_mask(seq_q: int, seq_kv: int, dtype=np.float64) -> np.ndarray:
    """Additive causal mask, -1e38 above the (bottom-right aligned) diagonal.

    Restates mlx_primitives/utils/masking.py:14-66 (triu with k = Sk - Sq + 1).
    """
    full = np.full((seq_q, seq_kv), ATTENTION_MASK_VALUE, dtype=dtype)
    return np.triu(full, k=seq_kv - seq_q + 1)


def _softmax_last(x: np.ndarray) -> np.ndarray:
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=-1, keepdims=True)


def dense_attention_bhsd(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, causal: bool,
    head_chunk: Optional[int] = None,
) -> np.ndarray:
    """BHSD dense attention: softmax(q k^T * scale + causal mask) v.

    Restates the BHSD fallback branch mlx_primitives/attention/flash.py:172-192
    (no epsilon; exact softmax). ``head_chunk`` evaluates heads in groups to
    bound memory; it does not change the arithmetic.
    """
    bsz, heads, seq_q, dim = q.shape
    seq_kv = k.shape[2]
    out = np.empty((bsz, heads, seq_q, v.shape[3]), dtype=q.dtype)
    step = head_chunk or heads
    mask = causal_additive_mask(seq_q, seq_kv, q.dtype) if causal else None
    for h0 in range(0, heads, step):
        qs, ks, vs = q[:, h0:h0 + step], k[:, h0:h0 + step], v[:, h0:h0 + step]
        scores = np.matmul(qs, np.swapaxes(ks, -1, -2)) * q.dtype.type(scale)
        if mask is not None:
            scores = scores + mask[None, None]
        out[:, h0:h0 + step] = np.matmul(_softmax_last(scores), vs)
    return out


def sdpa_causal_keep(seq_q: int, seq_kv: int) -> np.ndarray:
    """(Sq, Sk) visibility of ``mx.fast.scaled_dot_product_attention(mask="causal")``.

    The reference's default routes (attention/flash.py:177-181 BHSD, 211-215 and
    479-506 short BSHD, 221-235 long BSHD; kernels/fused_rope_attention.py:716-727)
    hand the causal mask to MLX's SDPA (MLX >= 0.20.0, pyproject.toml:37; not
    under /root/reference). Its causal rule aligns the diagonal at the bottom
    right when the keys outnumber the queries, so the last query sees every key
    (the intent stated at utils/masking.py:52-56, triu with k = Sk - Sq + 1), and
    at the top left otherwise (offset max(0, Sk - Sq)): key j is visible to
    query i iff j <= i + max(0, Sk - Sq). For Sq <= Sk this is exactly
    create_causal_mask (causal_additive_mask below); for Sq > Sk it is the
    top-left rule of the tiled path (_online_softmax.py:149-154), where the
    dense fallback's (Sq, Sq) mask (flash.py:188) cannot broadcast.
    """
    off = max(0, seq_kv - seq_q)
    return np.arange(seq_kv)[None, :] <= np.arange(seq_q)[:, None] + off


def sdpa_attention(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, causal: bool,
) -> np.ndarray:
    """BHSD exact-softmax attention with SDPA's causal rule (sdpa_causal_keep).

    The arithmetic of the reference's SDPA routes (no epsilon); q (B, H, Sq, D),
    k / v (B, H, Sk, D).
    """
    scores = np.matmul(q, np.swapaxes(k, -1, -2)) * q.dtype.type(scale)
    if causal:
        keep = sdpa_causal_keep(q.shape[2], k.shape[2])
        scores = np.where(keep[None, None], scores, -np.inf)
    return np.matmul(_softmax_last(scores), v)


def flash_attention_default_route(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: Optional[float] = None,
    causal: bool = True, layout: str = "BSHD",
) -> np.ndarray:
    """flash_attention on the reference's default route (use_metal=True, no
    dropout): every size and layout goes to SDPA (flash.py:177-181, 211-235,
    479-506), so the result is sdpa_attention in the caller's layout."""
    layout = getattr(layout, "value", layout)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if layout == "BHSD":
        return sdpa_attention(q, k, v, scale, causal)
    t = lambda x: np.ascontiguousarray(np.transpose(x, (0, 2, 1, 3)))
    return np.transpose(sdpa_attention(t(q), t(k), t(v), scale, causal), (0, 2, 1, 3))


def flash_attention(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: Optional[float] = None,
    causal: bool = True, block_q: int = 32, block_kv: int = 32, layout: str = "BSHD",
) -> np.ndarray:
    """flash_attention restated on the reference's CPU route (use_metal=False).

    mlx_primitives/attention/flash.py:52-254: BHSD goes to the dense branch
    (172-192); BSHD goes to the tiled path (254 -> 257-316). The reference's
    short-sequence shortcut (211-215) computes the same attention without the
    epsilon; the oracle keeps the tiled path for every BSHD size. With Sq == Sk
    (every causal BASELINE configuration) this equals the default route
    (flash_attention_default_route); for causal Sq != Sk the routes differ
    (the tiled path is top-left aligned, SDPA bottom-right when Sk > Sq).
    """
    layout = getattr(layout, "value", layout)
    dim = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(dim)
    if layout == "BHSD":
        return dense_attention_bhsd(q, k, v, scale, causal)
    return tiled_flash_attention(q, k, v, scale, causal, block_q, block_kv)


def windowed_chunk_attention(
    q: np.ndarray, k_chunk: np.ndarray, v_chunk: np.ndarray, scale: float, causal: bool,
    q_offset: int, kv_offset: int, window_size: int,
) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Chunk attention under the window mask |q - kv| <= W (and kv <= q if causal).

    Restates mlx_primitives/attention/sliding_window.py:447-511.
    """
    seq_q = q.shape[1]
    chunk = k_chunk.shape[1]
    scores = _bhqk(q, k_chunk) * q.dtype.type(scale)
    q_pos = np.arange(seq_q) + q_offset
    kv_pos = np.arange(chunk) + kv_offset
    keep = np.abs(q_pos[:, None] - kv_pos[None, :]) <= window_size
    if causal:
        keep = keep & (kv_pos[None, :] <= q_pos[:, None])
    scores = np.where(keep[None, :, None, :], scores, q.dtype.type(ATTENTION_MASK_VALUE))
    chunk_max = np.max(scores, axis=-1)
    e = np.exp(scores - chunk_max[..., None])
    return _bqhd(e, v_chunk), chunk_max, np.sum(e, axis=-1)


def tiled_sliding_window_attention(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, window_size: int, scale: float,
    causal: bool, block_q: int = 32,
) -> np.ndarray:
    """Tiled sliding-window attention (BSHD).

    Restates mlx_primitives/attention/sliding_window.py:363-444: q blocks of
    block_q; KV from max(0, q_start - W) to q_end (causal) or
    min(S, q_end + W) in steps of block_q; o / (l + 1e-6).
    """
    bsz, seq_len, heads, dim = q.shape
    dt = q.dtype.type
    blocks = []
    for q_start in range(0, seq_len, block_q):
        q_end = min(q_start + block_q, seq_len)
        qb = q[:, q_start:q_end]
        nq = q_end - q_start
        m_i = np.full((bsz, nq, heads), ATTENTION_MASK_VALUE, dtype=q.dtype)
        l_i = np.zeros((bsz, nq, heads), dtype=q.dtype)
        o_i = np.zeros((bsz, nq, heads, dim), dtype=q.dtype)
        kv_start = max(0, q_start - window_size)
        kv_end = q_end if causal else min(seq_len, q_end + window_size)
        for kb in range(kv_start, kv_end, block_q):
            ke = min(kb + block_q, kv_end)
            co, cm, cl = windowed_chunk_attention(
                qb, k[:, kb:ke], v[:, kb:ke], scale, causal, q_start, kb, window_size)
            o_i, m_i, l_i = online_softmax_merge(o_i, m_i, l_i, co, cm, cl)
        blocks.append(o_i / (l_i[..., None] + dt(SOFTMAX_EPSILON)))
    return np.concatenate(blocks, axis=1)


def sliding_window_attention(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, window_size: int,
    scale: Optional[float] = None, causal: bool = True,
) -> np.ndarray:
    """sliding_window_attention on the reference's CPU route.

    mlx_primitives/attention/sliding_window.py:227-313 -> tiled path (311-313).
    """
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    return tiled_sliding_window_attention(q, k, v, window_size, scale, causal)


def chunked_cross_attention_impl(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, chunk_size: int, scale: float, causal: bool,
) -> np.ndarray:
    """KV-chunked cross attention with full-Q accumulators.

    Restates mlx_primitives/attention/chunked.py:129-169.
    """
    bsz, seq_q, heads, dim = q.shape
    seq_kv = k.shape[1]
    dt = q.dtype.type
    acc = np.zeros((bsz, seq_q, heads, dim), dtype=q.dtype)
    mx_ = np.full((bsz, seq_q, heads), ATTENTION_MASK_VALUE, dtype=q.dtype)
    sm = np.zeros((bsz, seq_q, heads), dtype=q.dtype)
    for cs in range(0, seq_kv, chunk_size):
        ce = min(cs + chunk_size, seq_kv)
        co, cm, cl = compute_chunk_attention(
            q, k[:, cs:ce], v[:, cs:ce], scale, causal=causal, q_offset=0, kv_offset=cs)
        acc, mx_, sm = online_softmax_merge(acc, mx_, sm, co, cm, cl)
    return acc / (sm[..., None] + dt(SOFTMAX_EPSILON))


def reference_cross_attention(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, causal: bool,
) -> np.ndarray:
    """Dense cross attention (top-left causal, -1e38 mask, exact softmax).

    Restates mlx_primitives/attention/chunked.py:172-203, the branch
    chunked_cross_attention takes when Skv <= chunk_size (113-114): key j is
    visible to query i iff j <= i (absolute positions from 0 on both sides).
    """
    qt, kt, vt = (np.transpose(x, (0, 2, 1, 3)) for x in (q, k, v))
    scores = np.matmul(qt, np.swapaxes(kt, -1, -2)) * q.dtype.type(scale)
    if causal:
        keep = np.arange(k.shape[1])[None, :] <= np.arange(q.shape[1])[:, None]
        scores = np.where(keep[None, None], scores, q.dtype.type(ATTENTION_MASK_VALUE))
    return np.transpose(np.matmul(_softmax_last(scores), vt), (0, 2, 1, 3))


def chunked_cross_attention(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, chunk_size: int = 1024,
    scale: Optional[float] = None, causal: bool = False,
) -> np.ndarray:
    """chunked_cross_attention on the reference's CPU route.

    mlx_primitives/attention/chunked.py:43-126: dense when Skv <= chunk_size
    (113-114), else the chunk loop (126).
    """
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if k.shape[1] <= chunk_size:
        return reference_cross_attention(q, k, v, scale, causal)
    return chunked_cross_attention_impl(q, k, v, chunk_size, scale, causal)


def attention_rows(
    q_rows: np.ndarray, k: np.ndarray, v: np.ndarray, q_pos: np.ndarray, scale: float,
    causal: bool, window_left: int = -1, window_right: int = -1, eps: float = SOFTMAX_EPSILON,
) -> np.ndarray:
    """Exact attention for selected query rows of one (batch, head).

    q_rows (n, D) at absolute positions q_pos (n,), k/v (Sk, D). Mask as the
    reference's masks at kv <= q (causal), q - kv <= window_left and
    kv - q <= window_right (window of sliding_window.py:151-157), with the
    tiled path's o / (l + eps) normaliser. Used for sampled full-size checks.
    """
    scores = (q_rows @ k.T) * scale
    kv = np.arange(k.shape[0])[None, :]
    qp = q_pos[:, None]
    keep = np.ones(scores.shape, dtype=bool)
    if causal:
        keep &= kv <= qp
    if window_left >= 0:
        keep &= (qp - kv) <= window_left
    if window_right >= 0 and not causal:
        keep &= (kv - qp) <= window_right
    scores = np.where(keep, scores, -np.inf)
    m = np.max(scores, axis=-1, keepdims=True)
    e = np.exp(scores - m)
    return (e @ v) / (np.sum(e, axis=-1, keepdims=True) + eps)

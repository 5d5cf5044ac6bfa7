"""Flash attention on MI355X: the mlx-primitives ``flash_attention`` API.

Drop-in for mlx_primitives/attention/flash.py (flash_attention 52-254,
FlashAttention 581-647, get_optimal_flash_config 650-688): same signature,
same validation errors and messages, same defaults. Every call runs the gfx950
MFMA kernel of libmpx_attn.so (exact online softmax, causal mask by index
arithmetic, BSHD and BHSD through strides).

Arguments that only steer the reference's internal dispatch are accepted and
do not change the result: ``block_q``/``block_kv`` (the kernel has its own
tiles, as the reference's SDPA route ignores them too) and ``use_metal``
(there is one GPU path).
"""

from __future__ import annotations

import math
from typing import Optional, Tuple, Union

import torch

from mlx_primitives.attention._launch import check_dropout_p, run_attention
from mlx_primitives.constants import Layout


def _validate(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layout,
              enable_gqa: bool = False) -> Layout:
    # Mirrors mlx_primitives/attention/flash.py:123-169 (messages included).
    if q.ndim != 4:
        raise ValueError(f"Expected 4D tensors, got {q.ndim}D")
    if k.ndim != 4:
        raise ValueError(f"Expected K to be 4D tensor, got {k.ndim}D")
    if v.ndim != 4:
        raise ValueError(f"Expected V to be 4D tensor, got {v.ndim}D")
    if isinstance(layout, str) and layout not in (Layout.BSHD.value, Layout.BHSD.value):
        raise ValueError(
            f"layout must be Layout.BSHD or Layout.BHSD (or 'BSHD'/'BHSD'), got '{layout}'")
    layout = Layout(layout) if isinstance(layout, str) else layout
    if layout == Layout.BSHD:
        qb, qs, qh, qd = q.shape
        kb, ks, kh, kd = k.shape
        vb, vs, vh, vd = v.shape
    else:
        qb, qh, qs, qd = q.shape
        kb, kh, ks, kd = k.shape
        vb, vh, vs, vd = v.shape
    if qb != kb or qb != vb:
        raise ValueError(f"Batch size mismatch: Q={qb}, K={kb}, V={vb}")
    if enable_gqa:
        if kh != vh or kh == 0 or qh % kh != 0:
            raise ValueError(
                f"enable_gqa needs K and V with equal head counts dividing Q's: Q={qh}, "
                f"K={kh}, V={vh}")
    elif qh != kh or qh != vh:
        raise ValueError(f"Number of heads mismatch: Q={qh}, K={kh}, V={vh}")
    if qd != kd:
        raise ValueError(f"Head dimension mismatch between Q and K: Q={qd}, K={kd}")
    if ks != vs:
        raise ValueError(f"Sequence length mismatch between K and V: K={ks}, V={vs}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError(
            f"Q/K/V dtype mismatch: Q={q.dtype}, K={k.dtype}, V={v.dtype}. "
            "All tensors must have the same dtype to ensure numerical stability.")
    if vd != qd:
        # The reference would fail inside the kernel; the MI355X kernel needs
        # equal q/k/v head dims.
        raise ValueError(f"Head dimension mismatch between Q and V: Q={qd}, V={vd}")
    return layout


def flash_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: Optional[float] = None,
    causal: bool = True,
    block_q: int = 32,
    block_kv: int = 32,
    use_metal: bool = True,
    dropout_p: float = 0.0,
    training: bool = True,
    layout: Union[str, Layout] = Layout.BSHD,
    *,
    enable_gqa: bool = False,
) -> torch.Tensor:
    """Exact attention, softmax(q k^T * scale [+ causal mask]) v, tiled on MFMA.

    Args mirror the reference (mlx_primitives/attention/flash.py:52-64):
      q, k, v: (B, S, H, D) for layout "BSHD" (default) or (B, H, S, D) for
        "BHSD"; float32, float16 or bfloat16 ROCm tensors of one dtype.
      scale: defaults to 1/sqrt(D).
      causal: key j visible to query i iff j <= i + max(0, Sk - Sq): the
        causal rule of the reference's default route, which hands
        mask="causal" to SDPA for every size and layout (flash.py:177-181,
        211-235, 479-506). With more keys than queries (a decode step over a
        cache) the diagonal sits at the bottom right, so the last query sees
        every key (utils/masking.py:52-56); otherwise it is the tiled path's
        top-left rule (kv <= q).
      block_q, block_kv, use_metal: accepted, no effect on the result.
      dropout_p, training: with dropout_p > 0 and training (BSHD), each
        attention weight is dropped with probability dropout_p and the kept
        ones scaled by 1 / (1 - dropout_p) (flash.py:202-205, 570-574). The
        keep mask is a counter-based hash of (seed, batch, head, query, key)
        evaluated inside the kernels (never stored); the seed comes from
        torch's default generator, and the backward regenerates the same
        mask. dropout_p must be in [0, 1). BHSD ignores dropout like the
        reference's BHSD branch.
      layout: "BSHD" / "BHSD" or Layout.
      enable_gqa: keyword-only extension (the reference requires equal head
        counts, flash.py:151-154): K and V may carry H_kv heads, H a multiple
        of H_kv; query head h attends with K/V head h // (H // H_kv).

    Returns a new tensor shaped like q, in q's dtype. Rows are normalised as
    o / (l + 1e-6), the reference tiled path's normaliser.
    """
    layout = _validate(q, k, v, layout, enable_gqa)
    head_dim = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    # Dropout applies to BSHD in training; BHSD ignores it, as the reference's
    # BHSD branch does (flash.py:161-191 returns before the dropout check).
    drop = dropout_p if (layout == Layout.BSHD and training and dropout_p > 0.0) else 0.0
    check_dropout_p(drop, "flash_attention")
    if causal:
        seq_q, seq_kv = ((q.shape[1], k.shape[1]) if layout == Layout.BSHD
                         else (q.shape[2], k.shape[2]))
        if seq_kv > seq_q:
            # bottom-right diagonal: j <= i + (Sk - Sq)
            return run_attention(q, k, v, layout, scale, causal=False,
                                 window_right=seq_kv - seq_q, dropout_p=drop)
    return run_attention(q, k, v, layout, scale, causal=causal, dropout_p=drop)


class FlashAttention:
    """Flash attention module (mlx_primitives/attention/flash.py:581-647).

    Always BSHD; block sizes default to 32 for head_dim <= 64, else 16, and are
    kept as attributes for API compatibility.
    """

    def __init__(self, num_heads: int, head_dim: int, causal: bool = True,
                 block_q: Optional[int] = None, block_kv: Optional[int] = None) -> None:
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.causal = causal
        self.scale = 1.0 / math.sqrt(head_dim)
        default_block = 32 if head_dim <= 64 else 16
        self.block_q = default_block if block_q is None else block_q
        self.block_kv = default_block if block_kv is None else block_kv

    def __call__(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        return flash_attention(q, k, v, scale=self.scale, causal=self.causal,
                               block_q=self.block_q, block_kv=self.block_kv)


def get_optimal_flash_config(seq_len: int, head_dim: int, num_heads: int) -> Tuple[int, int]:
    """Block-size heuristic of the reference (flash.py:650-688), kept for API parity.

    Three (block, head_dim + 4) fp32 tiles in a 26 KB budget; 32 for
    head_dim <= 64, 16 up to 128, 8 beyond, never above seq_len.
    """
    per_row_bytes = (head_dim + 4) * 4
    cap = (26000 // 3) // per_row_bytes
    if head_dim <= 64:
        base = 32
    elif head_dim <= 128:
        base = 16
    else:
        base = 8
    blk = min(base, cap, seq_len)
    return blk, blk

"""RoPE + flash attention on MI355X: the mlx-primitives fused RoPE API.

Drop-in for mlx_primitives/kernels/fused_rope_attention.py:
``fast_fused_rope_attention`` (637-733), ``fused_rope_attention`` (939-985)
and ``FusedRoPEFlashAttention`` (988-1109). K is rotated by the gfx950 RoPE
kernel into a scratch tensor; for 16-bit inputs with head_dim 32, 64 or 128
the flash kernel rotates Q itself as it loads it (as the reference's fused
kernel does, fused_rope_attention.py:766-800), otherwise Q goes through the
RoPE kernel too. Tensors are (batch, seq, heads, head_dim).

The two entry points mask differently, as in the reference:
  * ``fused_rope_attention`` / ``FusedRoPEFlashAttention`` follow the fused
    kernel's position rule (fused_rope_attention.py:125-131): query i at
    position q_offset + i sees key j at position kv_offset + j when
    kv_offset + j <= q_offset + i;
  * ``fast_fused_rope_attention`` rotates, then hands mask="causal" to SDPA
    (fused_rope_attention.py:716-727): the offsets move the rotation only and
    key j is visible to query i when j <= i + max(0, seq_kv - seq_q).
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from mlx_primitives import _native
from mlx_primitives.attention._launch import run_attention
from mlx_primitives.constants import Layout
from mlx_primitives.kernels.rope import precompute_rope_cache, rope


def _check_inputs(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    # fused_rope_attention.py:691-701
    if q.ndim != 4:
        raise ValueError(f"Q must be 4D (batch, seq_q, num_heads, head_dim), got {q.ndim}D")
    if k.ndim != 4:
        raise ValueError(f"K must be 4D (batch, seq_kv, num_heads, head_dim), got {k.ndim}D")
    if v.ndim != 4:
        raise ValueError(f"V must be 4D (batch, seq_kv, num_heads, head_dim), got {v.ndim}D")
    if q.shape[-1] % 2 != 0:
        raise ValueError(f"head_dim must be even for RoPE, got {q.shape[-1]}")
    if k.shape != v.shape:
        raise ValueError(f"K and V shapes must match, got {tuple(k.shape)} and {tuple(v.shape)}")
    if (q.shape[0], q.shape[2], q.shape[3]) != (k.shape[0], k.shape[2], k.shape[3]):
        raise ValueError(
            f"Q and K must agree in batch, heads and head_dim, got {tuple(q.shape)} and "
            f"{tuple(k.shape)}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError(f"Q/K/V dtype mismatch: {q.dtype}, {k.dtype}, {v.dtype}")


def _rope_attention(q, k, v, scale, cos_cache, sin_cache, rope_base, q_offset, kv_offset,
                    causal, position_rule: bool) -> torch.Tensor:
    """softmax(scale * rope(Q) rope(K)^T + mask) V on the gfx950 kernels, with
    the position rule (kv_offset + j <= q_offset + i) or SDPA's causal rule
    (j <= i + max(0, seq_kv - seq_q))."""
    _check_inputs(q, k, v)
    _native.require_no_grad(q, k, v)
    batch, seq_q, heads, dim = q.shape
    seq_kv = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(dim)
    if q_offset < 0 or kv_offset < 0:
        raise ValueError(f"position offsets must be >= 0, got {q_offset} and {kv_offset}")
    if cos_cache is None or sin_cache is None:
        max_pos = max(seq_q + q_offset, seq_kv + kv_offset)
        cos_cache, sin_cache = precompute_rope_cache(max_pos, dim, base=rope_base,
                                                     dtype=q.dtype, device=q.device)
    shift = q_offset - kv_offset if position_rule else max(0, seq_kv - seq_q)
    if causal and shift < 0:
        # kv_offset > q_offset: query rows i < -shift are placed before the
        # first key and see none; the reference kernel writes zeros for them
        # (its sum stays 0, fused_rope_attention.py:127-131, 176-186). Row
        # i >= -shift sees keys j <= i + shift: the top-left causal attention
        # of the rows from -shift on, rotated from position q_offset - shift.
        n0 = min(-shift, seq_q)
        out = torch.zeros_like(q)
        if n0 < seq_q:
            out[:, n0:] = _rope_attention(q[:, n0:], k, v, scale, cos_cache, sin_cache,
                                          rope_base, q_offset + n0, kv_offset, causal,
                                          position_rule)
        return out
    k_rot = rope(k, cos_cache, sin_cache, kv_offset)
    # kv_offset + j <= q_offset + i  <=>  j <= i + shift
    mask = (dict(causal=False) if not causal else
            dict(causal=True) if shift == 0 else dict(causal=False, window_right=shift))
    if q.dtype != torch.float32 and dim in (32, 64, 128):
        # Q is rotated by the attention kernel as it loads it (same arithmetic
        # and rounding as the RoPE kernel); caches go in as given.
        if seq_q + q_offset > cos_cache.shape[0]:
            raise ValueError(f"positions up to {seq_q + q_offset - 1} exceed the cache length "
                             f"{cos_cache.shape[0]}")
        cos_c, sin_c = (c if c.is_contiguous() and c.data_ptr() % 16 == 0 else c.contiguous()
                        for c in (cos_cache, sin_cache))
        return run_attention(q, k_rot, v, Layout.BSHD, scale,
                             q_rope=(cos_c, sin_c, q_offset), **mask)
    q_rot = rope(q, cos_cache, sin_cache, q_offset)
    return run_attention(q_rot, k_rot, v, Layout.BSHD, scale, **mask)


def fast_fused_rope_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: Optional[float] = None,
    cos_cache: Optional[torch.Tensor] = None,
    sin_cache: Optional[torch.Tensor] = None,
    rope_base: float = 10000.0,
    q_offset: int = 0,
    kv_offset: int = 0,
    causal: bool = False,
    use_tiled: Optional[bool] = None,
) -> torch.Tensor:
    """rope(Q) at q_offset, rope(K) at kv_offset, then attention with SDPA's
    causal rule (fused_rope_attention.py:637-733): with ``causal`` key j is
    visible to query i iff j <= i + max(0, seq_kv - seq_q), whatever the
    offsets.

    cos_cache / sin_cache: (positions, head_dim // 2), built with
    ``precompute_rope_cache(max(seq_q + q_offset, seq_kv + kv_offset),
    head_dim, rope_base, q.dtype)`` when not given (fused_rope_attention.py:
    703-709). ``use_tiled`` is ignored, as in the reference.
    """
    return _rope_attention(q, k, v, scale, cos_cache, sin_cache, rope_base, q_offset,
                           kv_offset, causal, position_rule=False)


def fused_rope_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: Optional[float] = None,
    cos_cache: Optional[torch.Tensor] = None,
    sin_cache: Optional[torch.Tensor] = None,
    rope_base: float = 10000.0,
    q_offset: int = 0,
    kv_offset: int = 0,
    causal: bool = False,
    use_metal: bool = True,
) -> torch.Tensor:
    """Fused RoPE + flash attention (fused_rope_attention.py:939-985) with the
    fused kernel's position rule: with ``causal`` key j is visible to query i
    iff kv_offset + j <= q_offset + i (fused_rope_attention.py:125-131).

    ``use_metal`` is accepted for signature compatibility; the gfx950 kernels
    always run (there is no CPU path).
    """
    return _rope_attention(q, k, v, scale, cos_cache, sin_cache, rope_base, q_offset,
                           kv_offset, causal, position_rule=True)


class FusedRoPEFlashAttention(torch.nn.Module):
    """Q/K/V projections, fused RoPE + flash attention, output projection
    (fused_rope_attention.py:988-1109). Returns (output, (k, v)) where (k, v)
    are the un-rotated keys and values, the cache for the next call. The
    attention kernels are forward-only: call the module under torch.no_grad()
    or torch.inference_mode()."""

    def __init__(self, dims: int, num_heads: int, head_dim: Optional[int] = None,
                 max_seq_len: int = 8192, rope_base: float = 10000.0, causal: bool = False,
                 bias: bool = False, device=None, dtype=None):
        super().__init__()
        self.dims = dims
        self.num_heads = num_heads
        self.head_dim = head_dim or dims // num_heads
        self.max_seq_len = max_seq_len
        self.rope_base = rope_base
        self.causal = causal
        self.scale = 1.0 / math.sqrt(self.head_dim)
        inner = self.num_heads * self.head_dim
        kw = dict(bias=bias, device=device, dtype=dtype)
        self.q_proj = torch.nn.Linear(dims, inner, **kw)
        self.k_proj = torch.nn.Linear(dims, inner, **kw)
        self.v_proj = torch.nn.Linear(dims, inner, **kw)
        self.out_proj = torch.nn.Linear(inner, dims, **kw)

    def forward(self, queries: torch.Tensor, keys: Optional[torch.Tensor] = None,
                values: Optional[torch.Tensor] = None,
                cache: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                offset: int = 0) -> Tuple[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
        if keys is None:
            keys = queries
        if values is None:
            values = keys
        batch, seq_q, _ = queries.shape
        seq_kv = keys.shape[1]
        q = self.q_proj(queries).reshape(batch, seq_q, self.num_heads, self.head_dim)
        k = self.k_proj(keys).reshape(batch, seq_kv, self.num_heads, self.head_dim)
        v = self.v_proj(values).reshape(batch, seq_kv, self.num_heads, self.head_dim)
        if cache is not None:
            k = torch.cat([cache[0], k], dim=1)
            v = torch.cat([cache[1], v], dim=1)
        out = fused_rope_attention(q, k, v, scale=self.scale, rope_base=self.rope_base,
                                   q_offset=offset, kv_offset=0, causal=self.causal)
        out = self.out_proj(out.reshape(batch, seq_q, -1))
        return out, (k, v)

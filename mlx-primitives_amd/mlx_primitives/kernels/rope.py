"""Rotary position embeddings on MI355X: the mlx-primitives ``rope`` API.

Drop-in for mlx_primitives/kernels/rope.py: ``precompute_rope_cache``
(223-255) builds the cos/sin tables, ``rope`` (451-497) applies the
half-split rotation through the gfx950 ``mpx_rope`` kernel (float32 math,
one rounding to the input dtype). Tensors are (batch, seq, heads, head_dim).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from mlx_primitives import _native


def precompute_rope_cache(seq_len: int, head_dim: int, base: float = 10000.0,
                          dtype: torch.dtype = torch.float32,
                          device=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables (seq_len, head_dim // 2): angle(t, i) = t * base**(-i / (head_dim/2)),
    evaluated in float32 and cast to ``dtype`` (rope.py:240-255)."""
    if head_dim % 2:
        raise ValueError(f"head_dim must be even for RoPE, got {head_dim}")
    half = head_dim // 2
    inv_freq = base ** (-torch.arange(0, half, dtype=torch.float32, device=device) / half)
    t = torch.arange(seq_len, dtype=torch.float32, device=device)
    freqs = torch.outer(t, inv_freq)
    return torch.cos(freqs).to(dtype), torch.sin(freqs).to(dtype)


def rope(x: torch.Tensor, cos_cache: torch.Tensor, sin_cache: torch.Tensor, offset: int = 0,
         use_metal: bool = True, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Rotate x (batch, seq, heads, head_dim) at positions offset .. offset+seq-1.

    ``use_metal`` is accepted for signature compatibility; the gfx950 kernel
    always runs. ``out`` (same shape and dtype as x) receives the result when
    given, else a new tensor is returned.
    """
    if x.ndim != 4:
        raise ValueError(f"Expected x of shape (batch, seq, heads, head_dim), got {x.ndim}D")
    B, S, H, D = x.shape
    if D % 2:
        raise ValueError(f"head_dim must be even for RoPE, got {D}")
    if D % 16:
        raise NotImplementedError(
            f"rope: the MI355X kernel needs head_dim to be a multiple of 16, got {D}")
    half = D // 2
    if cos_cache.shape != sin_cache.shape or cos_cache.ndim != 2 or cos_cache.shape[1] != half:
        raise ValueError(
            f"cos/sin caches must both be (positions, {half}); got {tuple(cos_cache.shape)} "
            f"and {tuple(sin_cache.shape)}")
    if offset < 0 or offset + S > cos_cache.shape[0]:
        raise ValueError(
            f"positions {offset}..{offset + S - 1} exceed the cache's {cos_cache.shape[0]} rows")
    _native.require_device(x, cos_cache, sin_cache)
    _native.require_no_grad(x, cos_cache, sin_cache)
    cos_cache = cos_cache.contiguous()
    sin_cache = sin_cache.contiguous()
    vec = 4 if x.dtype == torch.float32 else 8
    if x.stride(-1) != 1 or any(st % vec for st in x.stride()[:3]) or x.data_ptr() % 16:
        x = x.contiguous()
    if out is None:
        out = torch.empty((B, S, H, D), dtype=x.dtype, device=x.device)
    elif out.shape != x.shape or out.dtype != x.dtype or out.stride(-1) != 1:
        raise ValueError("out must match x's shape and dtype with a contiguous last dimension")
    _native.rope(x, out, cos_cache, sin_cache, offset)
    return out


def rope_at(x: torch.Tensor, cos_cache: torch.Tensor, sin_cache: torch.Tensor,
            positions: torch.Tensor, out: Optional[torch.Tensor] = None, check: bool = True,
            errors: Optional[torch.Tensor] = None) -> torch.Tensor:
    """rope with a position per sequence (extension): row s of sequence b is
    rotated to positions[b] + s, the values rope(x[b:b+1], cos, sin,
    positions[b]) gives, for a whole decode batch in one kernel (each
    sequence's new query at the position it has reached).

    positions: int (batch,) tensor or sequence. With ``check`` the call waits
    and raises ValueError if a row's position falls outside the tables;
    otherwise such rows are left unwritten and ``errors`` (int32 (1,) device
    tensor, cleared here; a temporary when None) is set.
    """
    if x.ndim != 4:
        raise ValueError(f"Expected x of shape (batch, seq, heads, head_dim), got {x.ndim}D")
    B, S, H, D = x.shape
    if D % 2:
        raise ValueError(f"head_dim must be even for RoPE, got {D}")
    if D % 16:
        raise NotImplementedError(
            f"rope_at: the MI355X kernel needs head_dim to be a multiple of 16, got {D}")
    half = D // 2
    if cos_cache.shape != sin_cache.shape or cos_cache.ndim != 2 or cos_cache.shape[1] != half:
        raise ValueError(
            f"cos/sin caches must both be (positions, {half}); got {tuple(cos_cache.shape)} "
            f"and {tuple(sin_cache.shape)}")
    dev = _native.require_device(x, cos_cache, sin_cache)
    _native.require_no_grad(x, cos_cache, sin_cache)
    pos = torch.as_tensor(positions, dtype=torch.int32, device=dev).reshape(-1).contiguous()
    if pos.numel() != B:
        raise ValueError(f"positions must have {B} entries, got {pos.numel()}")
    cos_cache = cos_cache.contiguous()
    sin_cache = sin_cache.contiguous()
    vec = 4 if x.dtype == torch.float32 else 8
    if x.stride(-1) != 1 or any(st % vec for st in x.stride()[:3]) or x.data_ptr() % 16:
        x = x.contiguous()
    if out is None:
        out = torch.empty((B, S, H, D), dtype=x.dtype, device=x.device)
    elif out.shape != x.shape or out.dtype != x.dtype or out.stride(-1) != 1:
        raise ValueError("out must match x's shape and dtype with a contiguous last dimension")
    if errors is None:
        errors = torch.zeros(1, dtype=torch.int32, device=dev)
    else:
        if errors.dtype != torch.int32 or errors.numel() != 1 or errors.device != dev:
            raise ValueError("errors must be an int32 tensor of 1 entry on x's device")
        errors.zero_()
    _native.rope_at(x, out, cos_cache, sin_cache, pos, errors)
    if check and int(errors.item()):
        raise ValueError(f"a position in positions .. positions + {S - 1} lies outside the "
                         f"cache's {cos_cache.shape[0]} rows")
    return out

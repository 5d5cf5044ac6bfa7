"""Layout layer between the Python API and mpx_attn_fwd.

Turns BSHD / BHSD torch tensors into (batch, head, seq) element strides (no
transposes), pads unusual head dims up to a kernel size with zeros (exact:
zero dims add nothing to q.k and produce zero output columns that are sliced
off), allocates the output and calls the HIP kernel.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from mlx_primitives import _native
from mlx_primitives.constants import Layout

# Head dims of the kernels (forward, paged, dropout, backward); the reference's
# Metal kernel stops at METAL_ATTENTION_MAX_HEAD_DIM (128), its other routes
# take any D.
_KERNEL_HEAD_DIMS = (32, 64, 128, 256)
MAX_HEAD_DIM = _KERNEL_HEAD_DIMS[-1]


def kernel_head_dim(dim: int, limit: int = MAX_HEAD_DIM, what: str = "attention") -> int:
    """Smallest kernel head dim >= dim (inputs are zero-padded to it)."""
    for d in _KERNEL_HEAD_DIMS:
        if dim <= d <= limit:
            return d
    raise NotImplementedError(
        f"head_dim={dim} exceeds the MI355X {what} kernels' limit of {limit}")


def _prepare(x: torch.Tensor, dk: int) -> torch.Tensor:
    if x.shape[-1] != dk:
        return F.pad(x, (0, dk - x.shape[-1]))
    vec = 4 if x.dtype == torch.float32 else 8
    ok = (x.stride(-1) == 1 and x.data_ptr() % 16 == 0
          and all(s % vec == 0 for s in x.stride()[:-1]))
    return x if ok else x.contiguous()


def _bhs(x: torch.Tensor, layout: Layout):
    s = x.stride()
    return (s[0], s[2], s[1]) if layout == Layout.BSHD else (s[0], s[1], s[2])


def _needs_grad(*tensors: torch.Tensor) -> bool:
    return torch.is_grad_enabled() and any(t.requires_grad for t in tensors)


def _dims(q: torch.Tensor, k: torch.Tensor, layout: Layout):
    if layout == Layout.BSHD:
        B, Sq, H, D = q.shape
        return B, H, k.shape[2], Sq, k.shape[1], D
    B, H, Sq, D = q.shape
    return B, H, k.shape[1], Sq, k.shape[2], D


# The backward's schedule (_native.attn_bwd's stored_ds): None = the stored-dS
# schedule for the dropout backward where it applies and its workspace fits,
# True = the stored-dS schedule, False = recompute S and dP for dQ.
BWD_STORED_DS: Optional[bool] = None


class _FlashAttentionFn(torch.autograd.Function):
    """Flash forward that keeps each row's log-sum-exp, and the gfx950 backward
    (mpx_attn_bwd) that recomputes the probabilities from it. Inputs arrive
    padded to the kernel head dim; padding and slicing stay outside, where
    autograd differentiates them."""

    @staticmethod
    def forward(ctx, q, k, v, layout, scale, causal, window_left, window_right, dropout):
        B, H, H_kv, Sq, Sk, D = _dims(q, k, layout)
        o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        lse = torch.empty((B, H, Sq), dtype=torch.float32, device=q.device)
        _native.attn_fwd(q, k, v, o, _bhs(q, layout), _bhs(k, layout), _bhs(v, layout),
                         _bhs(o, layout), B, H, Sq, Sk, D, scale, causal, window_left,
                         window_right, H_kv=H_kv, lse=lse, dropout=dropout)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.cfg = (layout, scale, causal, window_left, window_right, dropout)
        return o

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dout):
        q, k, v, o, lse = ctx.saved_tensors
        layout, scale, causal, window_left, window_right, dropout = ctx.cfg
        B, H, H_kv, Sq, Sk, D = _dims(q, k, layout)
        dout = _prepare(dout, D)
        dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
        dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
        strides = [_bhs(x, layout) for x in (q, k, v, o, dout, dq, dk, dv)]
        _native.attn_bwd(q, k, v, o, dout, lse, dq, dk, dv, strides, B, H, H_kv, Sq, Sk, D,
                         scale, causal, window_left, window_right, dropout=dropout,
                         stored_ds=BWD_STORED_DS)
        return dq, dk, dv, None, None, None, None, None, None


def dropout_seed() -> int:
    """A 64-bit seed for the dropout keep mask, drawn from torch's default
    (CPU) generator, so torch.manual_seed makes the masks reproducible."""
    lo, hi = torch.randint(0, 2**32, (2,), dtype=torch.int64).tolist()
    return lo | (hi << 32)


def check_dropout_p(dropout_p: float, name: str) -> None:
    if not 0.0 <= dropout_p < 1.0:
        raise ValueError(f"{name}: dropout_p must be in [0, 1), got {dropout_p}")


def _attention_with_grad(q, k, v, layout, scale, causal, window_left, window_right,
                         dropout=None):
    if not scale > 0:
        raise NotImplementedError(
            "mlx_primitives (MI355X build) differentiates attention with scale > 0 only "
            f"(got scale={scale}); run it under torch.no_grad()")
    D = q.shape[-1]
    # Backward kernels: D = 64, 128 and 256.
    kernel_head_dim(D, MAX_HEAD_DIM, "backward")
    dk = 64 if D <= 64 else (128 if D <= 128 else 256)
    qk, kk, vk = (_prepare(x, dk) for x in (q, k, v))
    o = _FlashAttentionFn.apply(qk, kk, vk, layout, scale, causal, window_left, window_right,
                                dropout)
    return o[..., :D].contiguous() if dk != D else o


def run_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layout: Layout,
                  scale: float, causal: bool, window_left: int = -1,
                  window_right: int = -1, q_rope: Optional[tuple] = None,
                  dropout_p: float = 0.0, dropout_seed_value: Optional[int] = None
                  ) -> torch.Tensor:
    """Attention forward on the GPU kernel; returns a new tensor shaped like q.
    When autograd tracks q, k or v, the result is differentiable through the
    gfx950 backward kernels. q_rope = (cos_cache, sin_cache, q_offset) rotates Q
    inside the kernel (16-bit, D in 32/64/128, no gradients). dropout_p > 0
    drops attention weights by the kernels' counter-based keep mask, seeded by
    dropout_seed_value or else a fresh dropout_seed(); the backward regenerates
    the same mask."""
    _native.require_device(q, k, v)
    B, H, H_kv, Sq, Sk, D = _dims(q, k, layout)
    if q.numel() == 0:
        return torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = kernel_head_dim(D)
    dropout = None
    if dropout_p > 0.0:
        if dropout_seed_value is None and torch.cuda.is_current_stream_capturing():
            # The seed is a launch argument drawn on the host: a captured graph
            # would replay this one keep mask on every launch.
            raise RuntimeError(
                "mlx_primitives (MI355X build): attention dropout under HIP graph capture "
                "would reuse one keep mask on every replay; capture without dropout, or "
                "pass an explicit seed (run_attention(..., dropout_seed_value=...))")
        dropout = (float(dropout_p),
                   dropout_seed() if dropout_seed_value is None else int(dropout_seed_value))
    if q_rope is not None:
        if dk != D or q.dtype == torch.float32 or _needs_grad(q, k, v) or dropout:
            raise ValueError("in-kernel Q rotation needs 16-bit inputs, D in (32, 64, 128), "
                             "no gradients and no dropout")
    elif _needs_grad(q, k, v) or dropout:
        if _needs_grad(q, k, v):
            return _attention_with_grad(q, k, v, layout, scale, causal, window_left,
                                        window_right, dropout)
        # (the dropout kernels take D = 64, 128 or 256)
        dk = 64 if D <= 64 else (128 if D <= 128 else 256)
    qk, kk, vk = (_prepare(x, dk) for x in (q, k, v))
    out_shape = list(q.shape)
    out_shape[-1] = dk
    o = torch.empty(out_shape, dtype=q.dtype, device=q.device)
    _native.attn_fwd(qk, kk, vk, o, _bhs(qk, layout), _bhs(kk, layout), _bhs(vk, layout),
                     _bhs(o, layout), B, H, Sq, Sk, dk, scale, causal, window_left,
                     window_right, H_kv=H_kv, q_rope=q_rope, dropout=dropout)
    if dk != D:
        o = o[..., :D].contiguous()
    return o

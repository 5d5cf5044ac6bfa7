"""Layout layer between the Python API and mpx_attn_fwd.

Turns BSHD / BHSD torch tensors into (batch, head, seq) element strides (no
transposes), pads unusual head dims up to a kernel size with zeros (exact:
zero dims add nothing to q.k and produce zero output columns that are sliced
off), allocates the output and calls the HIP kernel.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from mlx_primitives import _native
from mlx_primitives.constants import METAL_ATTENTION_MAX_HEAD_DIM, Layout

_KERNEL_HEAD_DIMS = (32, 64, 128)


def kernel_head_dim(dim: int) -> int:
    for d in _KERNEL_HEAD_DIMS:
        if dim <= d:
            return d
    raise NotImplementedError(
        f"head_dim={dim} exceeds the MI355X kernel limit of {METAL_ATTENTION_MAX_HEAD_DIM}")


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


def run_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layout: Layout,
                  scale: float, causal: bool, window_left: int = -1,
                  window_right: int = -1) -> torch.Tensor:
    """Attention forward on the GPU kernel; returns a new tensor shaped like q."""
    _native.require_device(q, k, v)
    _native.require_no_grad(q, k, v)
    if layout == Layout.BSHD:
        B, Sq, H, D = q.shape
        Sk, H_kv = k.shape[1], k.shape[2]
    else:
        B, H, Sq, D = q.shape
        Sk, H_kv = k.shape[2], k.shape[1]
    if q.numel() == 0:
        return torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = kernel_head_dim(D)
    qk, kk, vk = (_prepare(x, dk) for x in (q, k, v))
    out_shape = list(q.shape)
    out_shape[-1] = dk
    o = torch.empty(out_shape, dtype=q.dtype, device=q.device)
    _native.attn_fwd(qk, kk, vk, o, _bhs(qk, layout), _bhs(kk, layout), _bhs(vk, layout),
                     _bhs(o, layout), B, H, Sq, Sk, dk, scale, causal, window_left,
                     window_right, H_kv=H_kv)
    if dk != D:
        o = o[..., :D].contiguous()
    return o

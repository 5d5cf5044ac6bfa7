"""ctypes binding of libmpx_attn.so (the gfx950 HIP kernels and their C ABI).

This is the launch layer that replaces the reference's
``mx.fast.metal_kernel`` dispatch (mlx_primitives/attention/flash.py:410-476,
mlx_primitives/kernels/_registry.py:36-165): the library is loaded once
(thread-safe), tensors are passed as raw device pointers plus element strides,
work is enqueued on torch's current HIP stream, and workspaces come from
torch's caching allocator. There is no CPU fallback: if the library is missing
or the tensors are not on a ROCm device, the call raises.
"""

from __future__ import annotations

import ctypes
import functools
import os
import threading
from typing import Optional, Sequence

import torch

# MPX_ATTN_LIB selects another build of the library (e.g. a tuning variant).
_LIB_PATH = os.environ.get("MPX_ATTN_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "_lib", "libmpx_attn.so")

MPX_OK = 0
MPX_EINVAL = -1
MPX_EUNSUPPORTED = -2
MPX_EHIP = -3

DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()

_i64p = ctypes.POINTER(ctypes.c_int64)


def library_path() -> str:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Load libmpx_attn.so once (double-checked under a lock)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(
                f"libmpx_attn.so not found at {_LIB_PATH}; build it with "
                "`python mlx-primitives_amd/build.py` (hipcc, gfx950)")
        lib = ctypes.CDLL(_LIB_PATH)
        lib.mpx_version.restype = ctypes.c_int
        lib.mpx_version.argtypes = []
        lib.mpx_last_error.restype = ctypes.c_char_p
        lib.mpx_last_error.argtypes = []
        lib.mpx_attn_fwd.restype = ctypes.c_int
        lib.mpx_attn_fwd.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            _i64p, _i64p, _i64p, _i64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ]
        lib.mpx_attn_fwd_gqa.restype = ctypes.c_int
        lib.mpx_attn_fwd_gqa.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            _i64p, _i64p, _i64p, _i64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ]
        lib.mpx_attn_fwd_lse.restype = ctypes.c_int
        lib.mpx_attn_fwd_lse.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            _i64p, _i64p, _i64p, _i64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ]
        lib.mpx_attn_fwd_rope.restype = ctypes.c_int
        lib.mpx_attn_fwd_rope.argtypes = [ctypes.c_void_p] * 4 + [_i64p] * 4 + [
            ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
                                 ctypes.c_void_p]
        lib.mpx_attn_bwd.restype = ctypes.c_int
        lib.mpx_attn_bwd.argtypes = [ctypes.c_void_p] * 9 + [_i64p] * 8 + [
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ]
        lib.mpx_attn_fwd_dropout.restype = ctypes.c_int
        lib.mpx_attn_fwd_dropout.argtypes = [ctypes.c_void_p] * 5 + [_i64p] * 4 + [
            ctypes.c_int] * 6 + [ctypes.c_float] + [ctypes.c_int] * 4 + [
            ctypes.c_float, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.mpx_attn_bwd_dropout.restype = ctypes.c_int
        lib.mpx_attn_bwd_dropout.argtypes = [ctypes.c_void_p] * 9 + [_i64p] * 8 + [
            ctypes.c_int] * 6 + [ctypes.c_float] + [ctypes.c_int] * 4 + [
            ctypes.c_float, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.mpx_attn_bwd_workspace_bytes.restype = ctypes.c_size_t
        lib.mpx_attn_bwd_workspace_bytes.argtypes = [ctypes.c_int] * 3
        lib.mpx_attn_bwd_ds_workspace_bytes.restype = ctypes.c_size_t
        lib.mpx_attn_bwd_ds_workspace_bytes.argtypes = [ctypes.c_int] * 9
        lib.mpx_attn_fwd_workspace_bytes.restype = ctypes.c_size_t
        lib.mpx_attn_fwd_workspace_bytes.argtypes = [ctypes.c_int] * 9
        lib.mpx_paged_decode.restype = ctypes.c_int
        lib.mpx_paged_decode.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p, _i64p, _i64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_float, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ]
        lib.mpx_paged_decode_gqa.restype = ctypes.c_int
        lib.mpx_paged_decode_gqa.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p, _i64p, _i64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
            ctypes.c_void_p,
        ]
        lib.mpx_paged_decode_workspace_bytes.restype = ctypes.c_size_t
        lib.mpx_paged_decode_workspace_bytes.argtypes = [ctypes.c_int] * 5
        lib.mpx_paged_prefill.restype = ctypes.c_int
        lib.mpx_paged_prefill.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p, _i64p, _i64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ]
        lib.mpx_paged_prefill_gqa.restype = ctypes.c_int
        lib.mpx_paged_prefill_gqa.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p, _i64p, _i64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ]
        lib.mpx_paged_prefill_workspace_bytes.restype = ctypes.c_size_t
        lib.mpx_paged_prefill_workspace_bytes.argtypes = [ctypes.c_int] * 8
        lib.mpx_rope.restype = ctypes.c_int
        lib.mpx_rope.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, _i64p, _i64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
        ]
        lib.mpx_rope_at.restype = ctypes.c_int
        lib.mpx_rope_at.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, _i64p, _i64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
        ]
        lib.mpx_kv_append_rope.restype = ctypes.c_int
        lib.mpx_kv_append_rope.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, _i64p, _i64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
            ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
        ]
        lib.mpx_kv_append.restype = ctypes.c_int
        lib.mpx_kv_append.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, _i64p, _i64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
        ]
        _lib = lib
        return lib


def _check(rc: int, what: str) -> None:
    if rc == MPX_OK:
        return
    msg = load().mpx_last_error().decode(errors="replace") or what
    if rc == MPX_EINVAL:
        raise ValueError(msg)
    if rc == MPX_EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def _strides(vals: Sequence[int]) -> ctypes.Array:
    return _strides_of(tuple(int(x) for x in vals))


@functools.lru_cache(maxsize=512)
def _strides_of(vals: tuple) -> ctypes.Array:
    # One int64[] per distinct stride tuple: the library only reads it during
    # the call, and nothing here writes it.
    return (ctypes.c_int64 * len(vals))(*vals)


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one ROCm device; the kernels have no CPU path."""
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            "mlx_primitives (MI355X build) runs on ROCm device tensors only; got "
            f"{dev.type} tensors")
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"all tensors must be on {dev}, got {t.device}")
    return dev


def require_no_grad(*tensors: Optional[torch.Tensor]) -> None:
    """For the forward-only kernels (paged attention, RoPE): refuse inputs that
    autograd would track, instead of returning outputs silently cut off from
    the graph."""
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise NotImplementedError(
            "mlx_primitives (MI355X build) implements the forward pass only; call it under "
            "torch.no_grad() or torch.inference_mode(), or pass detached tensors")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_ptr(dev: torch.device) -> int:
    """hipStream_t of torch's current stream on dev."""
    if _raw_stream is not None:
        return _raw_stream(dev.index if dev.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(dev).cuda_stream


@functools.lru_cache(maxsize=1024)
def _fwd_workspace_bytes(*args) -> int:
    # mpx_attn_fwd_workspace_bytes is a pure function of its arguments.
    return int(load().mpx_attn_fwd_workspace_bytes(*args))


def attn_fwd_workspace_bytes(B: int, H: int, Sq: int, Sk: int, D: int, causal: bool,
                             window_left: int, window_right: int, dtype: torch.dtype) -> int:
    return _fwd_workspace_bytes(B, H, Sq, Sk, D, int(causal), int(window_left),
                                int(window_right), dtype_code(dtype))


def attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
             q_strides: Sequence[int], k_strides: Sequence[int], v_strides: Sequence[int],
             o_strides: Sequence[int], B: int, H: int, Sq: int, Sk: int, D: int,
             scale: float, causal: bool, window_left: int = -1, window_right: int = -1,
             H_kv: Optional[int] = None, lse: Optional[torch.Tensor] = None,
             q_rope: Optional[tuple] = None, dropout: Optional[tuple] = None) -> None:
    """Enqueue mpx_attn_fwd_lse on the current stream (strides in (b, h, s) order;
    K/V carry H_kv heads, default H; lse: optional contiguous (B, H, Sq) float32
    that receives each row's base-2 log-sum-exp for the backward). With
    q_rope = (cos_cache, sin_cache, q_offset) the kernel rotates Q on load
    (mpx_attn_fwd_rope); with dropout = (dropout_p, seed) the weights are
    dropped by the counter-based keep mask (mpx_attn_fwd_dropout)."""
    lib = load()
    dev = require_device(q, k, v, o)
    code = dtype_code(q.dtype)
    if q_rope is not None:
        if lse is not None:
            raise ValueError("q_rope and lse cannot be combined")
        cos, sin, q_offset = q_rope
        require_device(q, cos, sin)
        ws_bytes = _fwd_workspace_bytes(B, H, Sq, Sk, D, int(causal), int(window_left),
                                        int(window_right), code)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
        rc = lib.mpx_attn_fwd_rope(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
            _strides(q_strides), _strides(k_strides), _strides(v_strides), _strides(o_strides),
            B, H, H if H_kv is None else H_kv, Sq, Sk, D, float(scale), int(causal),
            int(window_left), int(window_right), code, cos.data_ptr(), sin.data_ptr(),
            int(q_offset), int(cos.shape[0]), dtype_code(cos.dtype),
            ws.data_ptr() if ws is not None else None, ws_bytes, _stream_ptr(dev))
        _check(rc, "mpx_attn_fwd_rope failed")
        return
    if lse is not None:
        if (lse.dtype != torch.float32 or not lse.is_contiguous() or lse.device != dev
                or tuple(lse.shape) != (B, H, Sq)):
            raise ValueError("lse must be a contiguous (B, H, Sq) float32 tensor on the device")
    ws_bytes = _fwd_workspace_bytes(B, H, Sq, Sk, D, int(causal), int(window_left),
                                    int(window_right), code)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
            lse.data_ptr() if lse is not None else None,
            _strides(q_strides), _strides(k_strides), _strides(v_strides), _strides(o_strides),
            B, H, H if H_kv is None else H_kv, Sq, Sk, D, float(scale), int(causal),
            int(window_left), int(window_right), code)
    tail = (ws.data_ptr() if ws is not None else None, ws_bytes, _stream_ptr(dev))
    if dropout is not None:
        p, seed = dropout
        rc = lib.mpx_attn_fwd_dropout(*args, float(p), int(seed) & (2**64 - 1), *tail)
    else:
        rc = lib.mpx_attn_fwd_lse(*args, *tail)
    _check(rc, "mpx_attn_fwd failed")


_DS_LIMIT: dict = {}


def _ds_workspace_limit(dev: torch.device) -> int:
    """An eighth of the device's memory: the largest stored-dS workspace taken
    without being asked for."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _DS_LIMIT:
        _DS_LIMIT[idx] = torch.cuda.get_device_properties(idx).total_memory // 8
    return _DS_LIMIT[idx]


def attn_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
             dout: torch.Tensor, lse: torch.Tensor, dq: torch.Tensor, dk: torch.Tensor,
             dv: torch.Tensor, strides: Sequence[Sequence[int]], B: int, H: int, H_kv: int,
             Sq: int, Sk: int, D: int, scale: float, causal: bool, window_left: int = -1,
             window_right: int = -1, dropout: Optional[tuple] = None,
             stored_ds: Optional[bool] = None) -> None:
    """Enqueue mpx_attn_bwd on the current stream. ``strides`` holds the (b, h, s)
    element strides of q, k, v, o, dout, dq, dk, dv in that order; dropout =
    (dropout_p, seed) of the forward (mpx_attn_bwd_dropout).

    stored_ds: the stored-dS schedule (mpx_attn_bwd_ds_workspace_bytes) or the
    recomputing one. None takes the stored one for the dropout backward (whose
    dQ kernel would otherwise regenerate the keep mask as well: 6% faster over
    forward and backward at the headline shape), where the problem has it and
    its workspace is at most an eighth of the device's memory and can be
    allocated; without dropout the two schedules run level and the recomputing
    one needs no workspace. False keeps the recomputing schedule; True requires
    the stored one."""
    lib = load()
    dev = require_device(q, k, v, o, dout, lse, dq, dk, dv)
    code = dtype_code(q.dtype)
    ws_bytes = int(lib.mpx_attn_bwd_workspace_bytes(B, H, Sq))
    ws = None
    if stored_ds or (stored_ds is None and dropout is not None):
        ds_bytes = int(lib.mpx_attn_bwd_ds_workspace_bytes(
            B, H, Sq, Sk, D, code, int(causal), int(window_left), int(window_right)))
        if stored_ds and not ds_bytes:
            raise ValueError("mpx_attn_bwd: no stored-dS schedule for this problem")
        if ds_bytes and (stored_ds or ds_bytes <= _ds_workspace_limit(dev)):
            try:
                ws = torch.empty(ds_bytes, dtype=torch.uint8, device=dev)
                ws_bytes = ds_bytes
            except torch.OutOfMemoryError:
                if stored_ds:
                    raise
    if ws is None:
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), dout.data_ptr(),
            lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
            *[_strides(s) for s in strides],
            B, H, H_kv, Sq, Sk, D, float(scale), int(causal), int(window_left),
            int(window_right), code)
    tail = (ws.data_ptr(), ws_bytes, _stream_ptr(dev))
    if dropout is not None:
        p, seed = dropout
        rc = lib.mpx_attn_bwd_dropout(*args, float(p), int(seed) & (2**64 - 1), *tail)
    else:
        rc = lib.mpx_attn_bwd(*args, *tail)
    _check(rc, "mpx_attn_bwd failed")


def paged_decode(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                 block_tables: torch.Tensor, context_lens: torch.Tensor,
                 alibi_slopes: Optional[torch.Tensor], o: torch.Tensor,
                 q_strides: Sequence[int], o_strides: Sequence[int], B: int, H: int, D: int,
                 num_blocks: int, block_size: int, max_blocks: int, scale: float,
                 H_kv: Optional[int] = None) -> None:
    """Enqueue mpx_paged_decode_gqa on the current stream (pools carry H_kv heads)."""
    lib = load()
    dev = require_device(q, k_pool, v_pool, block_tables, context_lens, o)
    code = dtype_code(q.dtype)
    ws_bytes = int(lib.mpx_paged_decode_workspace_bytes(B, H, D, block_size, max_blocks))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    rc = lib.mpx_paged_decode_gqa(
        q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), block_tables.data_ptr(),
        context_lens.data_ptr(), alibi_slopes.data_ptr() if alibi_slopes is not None else None,
        o.data_ptr(), _strides(q_strides), _strides(o_strides), B, H,
        H if H_kv is None else H_kv, D, num_blocks, block_size, max_blocks, float(scale), code,
        ws.data_ptr(), ws.numel(), _stream_ptr(dev))
    _check(rc, "mpx_paged_decode failed")


def paged_prefill(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                  block_tables: torch.Tensor, context_lens: torch.Tensor,
                  alibi_slopes: Optional[torch.Tensor], o: torch.Tensor,
                  q_strides: Sequence[int], o_strides: Sequence[int], B: int, Sq: int, H: int,
                  D: int, num_blocks: int, block_size: int, max_blocks: int, scale: float,
                  causal: bool, H_kv: Optional[int] = None) -> None:
    """Enqueue mpx_paged_prefill_gqa on the current stream (strides in (b, h, s)
    order; pools carry H_kv heads)."""
    lib = load()
    dev = require_device(q, k_pool, v_pool, block_tables, context_lens, o)
    code = dtype_code(q.dtype)
    ws_bytes = int(lib.mpx_paged_prefill_workspace_bytes(B, Sq, H, D, block_size, max_blocks,
                                                          int(causal), code))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    rc = lib.mpx_paged_prefill_gqa(
        q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), block_tables.data_ptr(),
        context_lens.data_ptr(), alibi_slopes.data_ptr() if alibi_slopes is not None else None,
        o.data_ptr(), _strides(q_strides), _strides(o_strides), B, Sq, H,
        H if H_kv is None else H_kv, D, num_blocks, block_size, max_blocks, float(scale),
        int(causal), code,
        ws.data_ptr() if ws is not None else None, ws_bytes, _stream_ptr(dev))
    _check(rc, "mpx_paged_prefill failed")


def kv_append(k: torch.Tensor, v: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
              block_tables: torch.Tensor, start_pos: torch.Tensor, n_tokens: torch.Tensor,
              errors: torch.Tensor, k_strides: Sequence[int], v_strides: Sequence[int], B: int,
              T: int, H: int, D: int, num_blocks: int, block_size: int, max_blocks: int) -> None:
    """Enqueue mpx_kv_append on the current stream (strides in (b, t, h) order)."""
    lib = load()
    dev = require_device(k, v, k_pool, v_pool, block_tables, start_pos, n_tokens, errors)
    rc = lib.mpx_kv_append(
        k.data_ptr(), v.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(),
        block_tables.data_ptr(), start_pos.data_ptr(), n_tokens.data_ptr(),
        _strides(k_strides), _strides(v_strides), B, T, H, D, num_blocks, block_size, max_blocks,
        dtype_code(k_pool.dtype), errors.data_ptr(), _stream_ptr(dev))
    _check(rc, "mpx_kv_append failed")


def kv_append_rope(k: torch.Tensor, v: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                   block_tables: torch.Tensor, start_pos: torch.Tensor, n_tokens: torch.Tensor,
                   errors: torch.Tensor, k_strides: Sequence[int], v_strides: Sequence[int],
                   B: int, T: int, H: int, D: int, num_blocks: int, block_size: int,
                   max_blocks: int, cos_cache: torch.Tensor, sin_cache: torch.Tensor) -> None:
    """Enqueue mpx_kv_append_rope on the current stream (strides in (b, t, h) order)."""
    lib = load()
    dev = require_device(k, v, k_pool, v_pool, block_tables, start_pos, n_tokens, errors,
                         cos_cache, sin_cache)
    rc = lib.mpx_kv_append_rope(
        k.data_ptr(), v.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(),
        block_tables.data_ptr(), start_pos.data_ptr(), n_tokens.data_ptr(),
        _strides(k_strides), _strides(v_strides), B, T, H, D, num_blocks, block_size, max_blocks,
        dtype_code(k_pool.dtype), cos_cache.data_ptr(), sin_cache.data_ptr(),
        cos_cache.shape[0], dtype_code(cos_cache.dtype), errors.data_ptr(), _stream_ptr(dev))
    _check(rc, "mpx_kv_append_rope failed")


def rope_at(x: torch.Tensor, out: torch.Tensor, cos_cache: torch.Tensor, sin_cache: torch.Tensor,
            positions: torch.Tensor, errors: torch.Tensor) -> None:
    """Enqueue mpx_rope_at on the current stream: row s of batch b at positions[b] + s."""
    lib = load()
    dev = require_device(x, out, cos_cache, sin_cache, positions, errors)
    B, S, H, D = x.shape
    rc = lib.mpx_rope_at(
        x.data_ptr(), out.data_ptr(), cos_cache.data_ptr(), sin_cache.data_ptr(),
        _strides((x.stride(0), x.stride(1), x.stride(2))),
        _strides((out.stride(0), out.stride(1), out.stride(2))),
        B, S, H, D, positions.data_ptr(), cos_cache.shape[0], dtype_code(x.dtype),
        dtype_code(cos_cache.dtype), errors.data_ptr(), _stream_ptr(dev))
    _check(rc, "mpx_rope_at failed")


def rope(x: torch.Tensor, out: torch.Tensor, cos_cache: torch.Tensor, sin_cache: torch.Tensor,
         offset: int) -> None:
    """Enqueue mpx_rope on the current stream: x, out (B, S, H, D), D contiguous."""
    lib = load()
    dev = require_device(x, out, cos_cache, sin_cache)
    B, S, H, D = x.shape
    rc = lib.mpx_rope(
        x.data_ptr(), out.data_ptr(), cos_cache.data_ptr(), sin_cache.data_ptr(),
        _strides((x.stride(0), x.stride(1), x.stride(2))),
        _strides((out.stride(0), out.stride(1), out.stride(2))),
        B, S, H, D, int(offset), cos_cache.shape[0], dtype_code(x.dtype),
        dtype_code(cos_cache.dtype), _stream_ptr(dev))
    _check(rc, "mpx_rope failed")

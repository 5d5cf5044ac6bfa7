"""mpx_paged_decode_noalloc (the paged decode that allocates nothing) through
the C ABI, against mpx_paged_decode_gqa with a caller workspace on the same
inputs: bit-identical outputs on consecutive calls, the second one smaller,
so stale partials of the first call left in the shared device scratch must
not leak into the second.
"""

import ctypes

import numpy as np
import pytest
import torch

from mlx_primitives import _native
import workloads as wl

pytestmark = pytest.mark.gpu

_i64p = ctypes.POINTER(ctypes.c_int64)
SCRATCH_BYTES = 32 << 20  # MPX_NOALLOC_SCRATCH_BYTES


def lib():
    lib = _native.load()
    fn = lib.mpx_paged_decode_noalloc
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p] * 7 + [_i64p, _i64p] + [ctypes.c_int] * 7 + [
        ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
    return lib


def strides(vals):
    return (ctypes.c_int64 * len(vals))(*vals)


def decode_both(q, kp, vp, tables, lens, slopes, H_kv, scale):
    """Run the workspace entry and the no-allocation entry; return both outputs."""
    L = lib()
    B, _, H, D = q.shape
    nb, bs = kp.shape[0], kp.shape[1]
    mb = tables.shape[1]
    code = _native.DTYPE_CODES[q.dtype]
    stream = torch.cuda.current_stream(q.device).cuda_stream
    qs = strides((q.stride(0), q.stride(2)))
    outs = []
    for noalloc in (False, True):
        o = torch.full_like(q, float("nan"))
        os_ = strides((o.stride(0), o.stride(2)))
        sp = slopes.data_ptr() if slopes is not None else None
        if noalloc:
            rc = L.mpx_paged_decode_noalloc(q.data_ptr(), kp.data_ptr(), vp.data_ptr(),
                                            tables.data_ptr(), lens.data_ptr(), sp, o.data_ptr(),
                                            qs, os_, B, H, H_kv, D, nb, bs, mb, scale, code,
                                            stream)
        else:
            ws_bytes = int(L.mpx_paged_decode_workspace_bytes(B, H, D, bs, mb))
            ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
            rc = L.mpx_paged_decode_gqa(q.data_ptr(), kp.data_ptr(), vp.data_ptr(),
                                        tables.data_ptr(), lens.data_ptr(), sp, o.data_ptr(),
                                        qs, os_, B, H, H_kv, D, nb, bs, mb, scale, code,
                                        ws.data_ptr(), ws.numel(), stream)
        assert rc == 0, L.mpx_last_error().decode()
        outs.append(o)
    torch.cuda.synchronize()
    return outs


def random_case(seed, B, H, H_kv, D, dtype, lens, bs=16, alibi=False, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    pages = [(n + bs - 1) // bs for n in lens]
    nb = sum(pages) + 3
    perm = torch.randperm(nb, generator=g)
    width = max(pages) + 1
    tables = torch.full((B, width), -1, dtype=torch.int32)
    off = 0
    for b, p in enumerate(pages):
        tables[b, :p] = perm[off:off + p]
        off += p
    q = torch.randn(B, 1, H, D, generator=g).to(dtype)
    kp = torch.randn(nb, bs, H_kv, D, generator=g).to(dtype)
    vp = torch.randn(nb, bs, H_kv, D, generator=g).to(dtype)
    slopes = (torch.rand(H, generator=g) * 0.1) if alibi else None
    mv = lambda x: None if x is None else x.to(device)
    return (mv(q), mv(kp), mv(vp), mv(tables), mv(torch.tensor(lens, dtype=torch.int32)),
            mv(slopes))


def test_noalloc_matches_workspace_entry_large_then_small(device):
    # Call 1: BASELINE config 4 (64 sequences, ctx U{512..8192}, H=32, D=128,
    # fp16): 17 MB of partials. Call 2: fewer, shorter sequences.
    inp = wl.make_paged(wl.CONFIGS["paged_decode_fp16"], device=device)
    a, b = decode_both(inp.q, inp.k_pool, inp.v_pool, inp.block_tables, inp.context_lens, None,
                       inp.q.shape[2], 1 / np.sqrt(128))
    assert torch.equal(a, b)
    q, kp, vp, t, l, s = random_case(1, 5, 32, 32, 128, torch.float16, [3000, 1, 777, 64, 2049],
                                     device=device)
    a, b = decode_both(q, kp, vp, t, l, s, 32, 1 / np.sqrt(128))
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_grouped_alibi_then_smaller(device, dtype):
    q, kp, vp, t, l, s = random_case(2, 6, 16, 4, 64, dtype, [5000, 130, 2, 4096, 17, 900],
                                     alibi=True, device=device)
    a, b = decode_both(q, kp, vp, t, l, s, 4, 0.125)
    assert torch.equal(a, b)
    q, kp, vp, t, l, s = random_case(3, 2, 16, 4, 64, dtype, [33, 600], alibi=True,
                                     device=device)
    a, b = decode_both(q, kp, vp, t, l, s, 4, 0.125)
    assert torch.equal(a, b)


def test_noalloc_rejects_calls_beyond_the_scratch(device):
    L = lib()
    # B * H * parts * (D + 2) * 4 bytes: 64 * 64 * 32 * 130 * 4 > 32 MiB
    B, H, D, bs, mb = 64, 64, 128, 16, 1024
    assert L.mpx_paged_decode_workspace_bytes(B, H, D, bs, mb) > SCRATCH_BYTES
    q = torch.zeros(B, 1, H, D, dtype=torch.float16, device=device)
    kp = torch.zeros(4, bs, H, D, dtype=torch.float16, device=device)
    tables = torch.full((B, mb), -1, dtype=torch.int32, device=device)
    lens = torch.zeros(B, dtype=torch.int32, device=device)
    rc = L.mpx_paged_decode_noalloc(q.data_ptr(), kp.data_ptr(), kp.data_ptr(), tables.data_ptr(),
                                    lens.data_ptr(), None, q.data_ptr(),
                                    strides((q.stride(0), q.stride(2))),
                                    strides((q.stride(0), q.stride(2))), B, H, H, D, 4, bs, mb,
                                    0.1, 1, torch.cuda.current_stream(device).cuda_stream)
    assert rc == _native.MPX_EINVAL
    assert "scratch" in L.mpx_last_error().decode()

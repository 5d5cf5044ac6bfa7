"""The reference-side ctypes binding of the integration guide works as written:
its code block is executed against the in-tree library and its results are
compared with the drop-in API on the same inputs (bit-identical: same kernels).
"""

import ctypes
import math
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def stub_namespace():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```python\n(.*?)```", text, re.S)
    code = [b for b in blocks if "ctypes.CDLL" in b]
    assert len(code) == 1
    from mlx_primitives import _native

    os.environ.setdefault("MPX_ATTN_LIB", _native.library_path())
    ns = {}
    exec(compile(code[0], "INTEGRATION.md", "exec"), ns)
    return ns


def test_stub_loads_and_binds():
    ns = stub_namespace()
    assert ns["_lib"].mpx_version() > 0
    with pytest.raises(ValueError):
        ns["_raise"](-1)
    for fn in ("flash_attention_fwd", "paged_attention_decode", "paged_attention_prefill",
               "store_kv", "rope", "flash_attention_fwd_lse", "flash_attention_bwd",
               "fused_rope_attention_fwd", "store_kv_rope", "rope_at",
               "flash_attention_dropout_fwd", "flash_attention_dropout_bwd"):
        assert callable(ns[fn]), fn


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["BSHD", "BHSD"])
def test_stub_flash_matches_api(device, layout):
    from mlx_primitives.attention import flash_attention

    ns = stub_namespace()
    g = torch.Generator().manual_seed(5)
    B, H, S, D = 2, 4, 200, 64
    shape = (B, S, H, D) if layout == "BSHD" else (B, H, S, D)
    q, k, v = (torch.randn(shape, generator=g).to(torch.bfloat16).to(device) for _ in range(3))
    o = torch.empty_like(q)
    bufs = []

    def alloc(n):
        bufs.append(torch.empty(n, dtype=torch.uint8, device=device))
        return bufs[-1].data_ptr()

    ns["flash_attention_fwd"](q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, S, S,
                              D, layout, ns["BF16"], 1 / math.sqrt(D), 1, alloc=alloc,
                              stream=torch.cuda.current_stream().cuda_stream)
    ref = flash_attention(q, k, v, causal=True, layout=layout)
    torch.cuda.synchronize()
    assert torch.equal(o, ref)


@pytest.mark.gpu
def test_stub_paged_matches_api(device):
    from mlx_primitives.cache import get_alibi_slopes, paged_attention

    ns = stub_namespace()
    g = torch.Generator().manual_seed(6)
    B, H, D, bs, nb = 3, 4, 128, 16, 12
    q = torch.randn(B, 1, H, D, generator=g).half().to(device)
    kp = torch.randn(nb, bs, H, D, generator=g).half().to(device)
    vp = torch.randn(nb, bs, H, D, generator=g).half().to(device)
    tables = torch.tensor([[5, 1, -1, -1], [0, 2, 3, 4], [11, -1, -1, -1]], dtype=torch.int32,
                          device=device)
    lens = torch.tensor([20, 64, 3], dtype=torch.int32, device=device)
    slopes = get_alibi_slopes(H).to(device)
    o = torch.empty_like(q)
    bufs = []

    def alloc(n):
        bufs.append(torch.empty(n, dtype=torch.uint8, device=device))
        return bufs[-1].data_ptr()

    ns["paged_attention_decode"](q.data_ptr(), kp.data_ptr(), vp.data_ptr(), tables.data_ptr(),
                                 lens.data_ptr(), o.data_ptr(), B, H, D, nb, bs, 4, ns["F16"],
                                 1 / math.sqrt(D), alibi_slopes=slopes.data_ptr(), alloc=alloc,
                                 stream=torch.cuda.current_stream().cuda_stream)
    ref = paged_attention(q, kp, vp, tables, lens, block_size=bs, alibi_slopes=slopes)
    torch.cuda.synchronize()
    assert torch.equal(o, ref)


@pytest.mark.gpu
def test_stub_paged_prefill_matches_api(device):
    from mlx_primitives.cache import get_alibi_slopes, paged_attention

    ns = stub_namespace()
    g = torch.Generator().manual_seed(7)
    B, Sq, H, D, bs, nb = 2, 40, 4, 64, 16, 10
    q = torch.randn(B, Sq, H, D, generator=g).to(torch.bfloat16).to(device)
    kp = torch.randn(nb, bs, H, D, generator=g).to(torch.bfloat16).to(device)
    vp = torch.randn(nb, bs, H, D, generator=g).to(torch.bfloat16).to(device)
    tables = torch.tensor([[3, 7, 1, -1], [0, 2, 9, 4]], dtype=torch.int32, device=device)
    lens = torch.tensor([45, 60], dtype=torch.int32, device=device)
    slopes = get_alibi_slopes(H).to(device)
    o = torch.empty_like(q)
    bufs = []

    def alloc(n):
        bufs.append(torch.empty(n, dtype=torch.uint8, device=device))
        return bufs[-1].data_ptr()

    ns["paged_attention_prefill"](q.data_ptr(), kp.data_ptr(), vp.data_ptr(), tables.data_ptr(),
                                  lens.data_ptr(), o.data_ptr(), B, Sq, H, D, nb, bs, 4,
                                  ns["BF16"], 1 / math.sqrt(D), causal=1,
                                  alibi_slopes=slopes.data_ptr(), alloc=alloc,
                                  stream=torch.cuda.current_stream().cuda_stream)
    ref = paged_attention(q, kp, vp, tables, lens, block_size=bs, causal=True,
                          alibi_slopes=slopes)
    torch.cuda.synchronize()
    assert torch.equal(o, ref)


@pytest.mark.gpu
def test_stub_store_kv_matches_api(device):
    from mlx_primitives.cache import store_kv

    ns = stub_namespace()
    g = torch.Generator().manual_seed(8)
    B, T, H, D, bs, nb = 2, 21, 4, 128, 16, 8
    k = torch.randn(B, T, H, D, generator=g).half().to(device)
    v = torch.randn(B, T, H, D, generator=g).half().to(device)
    tables = torch.tensor([[6, 1, 3], [0, 5, 7]], dtype=torch.int32, device=device)
    starts = torch.tensor([5, 16], dtype=torch.int32, device=device)
    counts = torch.tensor([21, 9], dtype=torch.int32, device=device)
    pools = [torch.zeros(nb, bs, H, D, dtype=torch.float16, device=device) for _ in range(4)]
    errors = torch.zeros(3, dtype=torch.int32, device=device)
    ns["store_kv"](k.data_ptr(), v.data_ptr(), pools[0].data_ptr(), pools[1].data_ptr(),
                   tables.data_ptr(), starts.data_ptr(), counts.data_ptr(), errors.data_ptr(),
                   B, T, H, D, nb, bs, 3, ns["F16"],
                   stream=torch.cuda.current_stream().cuda_stream)
    store_kv(pools[2], pools[3], tables, k, v, starts, counts)
    torch.cuda.synchronize()
    assert errors.tolist() == [0, 0, 0]
    assert torch.equal(pools[0], pools[2]) and torch.equal(pools[1], pools[3])
    assert pools[0].any()


@pytest.mark.gpu
def test_stub_store_kv_rope_and_rope_at_match_api(device):
    from mlx_primitives.cache import store_kv
    from mlx_primitives.kernels import precompute_rope_cache, rope_at

    ns = stub_namespace()
    g = torch.Generator().manual_seed(10)
    B, T, H, D, bs, nb = 2, 21, 4, 128, 16, 8
    k = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16).to(device)
    v = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16).to(device)
    cos, sin = precompute_rope_cache(64, D, device=device)
    tables = torch.tensor([[6, 1, 3], [0, 5, 7]], dtype=torch.int32, device=device)
    starts = torch.tensor([5, 16], dtype=torch.int32, device=device)
    counts = torch.tensor([21, 9], dtype=torch.int32, device=device)
    pools = [torch.zeros(nb, bs, H, D, dtype=torch.bfloat16, device=device) for _ in range(4)]
    errors = torch.zeros(4, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream().cuda_stream
    ns["store_kv_rope"](k.data_ptr(), v.data_ptr(), pools[0].data_ptr(), pools[1].data_ptr(),
                        tables.data_ptr(), starts.data_ptr(), counts.data_ptr(),
                        errors.data_ptr(), B, T, H, D, nb, bs, 3, ns["BF16"], cos.data_ptr(),
                        sin.data_ptr(), 64, ns["F32"], stream=stream)
    store_kv(pools[2], pools[3], tables, k, v, starts, counts, rope=(cos, sin))
    q = torch.randn(B, 1, H, D, generator=g).to(torch.bfloat16).to(device)
    q_out = torch.empty_like(q)
    pos = torch.tensor([25, 24], dtype=torch.int32, device=device)
    err1 = torch.zeros(1, dtype=torch.int32, device=device)
    ns["rope_at"](q.data_ptr(), q_out.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                  pos.data_ptr(), err1.data_ptr(), B, 1, H, D, 64, ns["BF16"], ns["F32"],
                  stream=stream)
    ref_q = rope_at(q, cos, sin, pos)
    torch.cuda.synchronize()
    assert errors.tolist() == [0, 0, 0, 0] and err1.item() == 0
    assert torch.equal(pools[0], pools[2]) and torch.equal(pools[1], pools[3])
    assert torch.equal(q_out, ref_q)


@pytest.mark.gpu
def test_stub_rope_matches_api(device):
    from mlx_primitives.kernels import precompute_rope_cache, rope

    ns = stub_namespace()
    g = torch.Generator().manual_seed(9)
    B, S, H, D = 2, 30, 4, 64
    x = torch.randn(B, S, H, D, generator=g).to(torch.bfloat16).to(device)
    cos, sin = precompute_rope_cache(40, D, dtype=torch.bfloat16, device=device)
    out = torch.empty_like(x)
    ns["rope"](x.data_ptr(), out.data_ptr(), cos.data_ptr(), sin.data_ptr(), B, S, H, D, 5, 40,
               ns["BF16"], ns["BF16"], stream=torch.cuda.current_stream().cuda_stream)
    ref = rope(x, cos, sin, 5)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["BSHD", "BHSD"])
def test_stub_backward_matches_autograd(device, layout):
    from mlx_primitives.attention import flash_attention

    ns = stub_namespace()
    g = torch.Generator().manual_seed(9)
    B, H, S, D = 2, 4, 300, 128
    shape = (B, S, H, D) if layout == "BSHD" else (B, H, S, D)
    q, k, v, do = (torch.randn(shape, generator=g).to(torch.bfloat16).to(device)
                   for _ in range(4))
    bufs = []

    def alloc(n):
        bufs.append(torch.empty(n, dtype=torch.uint8, device=device))
        return bufs[-1].data_ptr()

    st = torch.cuda.current_stream().cuda_stream
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, dtype=torch.float32, device=device)
    ns["flash_attention_fwd_lse"](q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                  lse.data_ptr(), B, H, S, S, D, layout, ns["BF16"],
                                  1 / math.sqrt(D), 1, alloc=alloc, stream=st)
    dq, dk, dv = (torch.empty_like(x) for x in (q, k, v))
    ns["flash_attention_bwd"](q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                              do.data_ptr(), lse.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                              dv.data_ptr(), B, H, S, S, D, layout, ns["BF16"],
                              1 / math.sqrt(D), 1, alloc=alloc, stream=st)
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    out = flash_attention(qg, kg, vg, causal=True, layout=layout)
    out.backward(do)
    torch.cuda.synchronize()
    assert torch.equal(o, out.detach())
    for mine, ref in ((dq, qg.grad), (dk, kg.grad), (dv, vg.grad)):
        assert torch.equal(mine, ref)


@pytest.mark.gpu
def test_stub_fused_rope_matches_api(device):
    from mlx_primitives.kernels import fused_rope_attention, precompute_rope_cache

    ns = stub_namespace()
    g = torch.Generator().manual_seed(11)
    B, S, H, D, q_off = 2, 150, 4, 128, 20
    q, k, v = (torch.randn(B, S, H, D, generator=g).to(torch.bfloat16).to(device)
               for _ in range(3))
    cos, sin = precompute_rope_cache(S + q_off, D, dtype=torch.bfloat16, device=device)
    st = torch.cuda.current_stream().cuda_stream
    kr = torch.empty_like(k)
    ns["rope"](k.data_ptr(), kr.data_ptr(), cos.data_ptr(), sin.data_ptr(), B, S, H, D, q_off,
               cos.shape[0], ns["BF16"], ns["BF16"], stream=st)
    o = torch.empty_like(q)
    bufs = []

    def alloc(n):
        bufs.append(torch.empty(n, dtype=torch.uint8, device=device))
        return bufs[-1].data_ptr()

    ns["fused_rope_attention_fwd"](q.data_ptr(), kr.data_ptr(), v.data_ptr(), o.data_ptr(),
                                   cos.data_ptr(), sin.data_ptr(), B, H, S, S, D, ns["BF16"],
                                   ns["BF16"], cos.shape[0], 1 / math.sqrt(D), q_offset=q_off,
                                   kv_offset=q_off, causal=1, alloc=alloc, stream=st)
    ref = fused_rope_attention(q, k, v, cos_cache=cos, sin_cache=sin, q_offset=q_off,
                               kv_offset=q_off, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(o, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("D", [64, 128])
def test_stub_dropout_matches_api(device, D):
    # (D = 128: both sides take the stored-dS backward)
    from mlx_primitives.attention._launch import run_attention
    from mlx_primitives.constants import Layout

    ns = stub_namespace()
    g = torch.Generator().manual_seed(11)
    B, H, S, p, seed = 2, 4, 260, 0.2, 0xDEADBEEF12345678
    q, k, v, do = (torch.randn((B, S, H, D), generator=g).to(torch.float16).to(device)
                   for _ in range(4))
    bufs = []

    def alloc(n):
        bufs.append(torch.empty(n, dtype=torch.uint8, device=device))
        return bufs[-1].data_ptr()

    st = torch.cuda.current_stream().cuda_stream
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, dtype=torch.float32, device=device)
    ns["flash_attention_dropout_fwd"](q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                      lse.data_ptr(), B, H, S, S, D, "BSHD", ns["F16"],
                                      1 / math.sqrt(D), 1, p, seed, alloc=alloc, stream=st)
    dq, dk, dv = (torch.empty_like(x) for x in (q, k, v))
    ns["flash_attention_dropout_bwd"](q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                      do.data_ptr(), lse.data_ptr(), dq.data_ptr(),
                                      dk.data_ptr(), dv.data_ptr(), B, H, S, S, D, "BSHD",
                                      ns["F16"], 1 / math.sqrt(D), 1, p, seed, alloc=alloc,
                                      stream=st)
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    out = run_attention(qg, kg, vg, Layout.BSHD, 1 / math.sqrt(D), True, dropout_p=p,
                        dropout_seed_value=seed)
    out.backward(do)
    torch.cuda.synchronize()
    assert torch.equal(o, out.detach())
    for mine, ref in ((dq, qg.grad), (dk, kg.grad), (dv, vg.grad)):
        assert torch.equal(mine, ref)

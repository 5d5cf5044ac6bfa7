"""HIP graph capture of the hot path: the kernels launch on the caller's
stream, take workspace from the caller (torch's allocator, the graph's pool
under capture) and clear no memory with memset nodes, so a serving loop can
capture them. Each graph is replayed several times with eager work and
synchronisations in between, and every replay is checked against the same
calls made eagerly (bit for bit).
"""

import pytest
import torch

from mlx_primitives.attention import flash_attention
from mlx_primitives.cache import paged_attention, store_kv

pytestmark = pytest.mark.gpu


def capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()  # warm the allocator and the library outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def test_flash_forward_graph(device):
    gen = torch.Generator(device=device).manual_seed(0)
    shape = (2, 8, 777, 128)
    q, k, v = (torch.randn(shape, device=device, generator=gen, dtype=torch.bfloat16)
               for _ in range(3))
    g, out = capture(lambda: flash_attention(q, k, v, causal=True, layout="BHSD"))
    for _ in range(4):
        for x in (q, k, v):
            x.copy_(torch.randn(shape, device=device, generator=gen, dtype=torch.bfloat16))
        g.replay()
        torch.cuda.synchronize()
        eager = flash_attention(q, k, v, causal=True, layout="BHSD")
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_decode_step_graph(device):
    # One serving step: append one token per sequence into its page, then decode.
    gen = torch.Generator(device=device).manual_seed(1)
    B, H, D, bs, pages = 4, 8, 128, 16, 64
    k_pool = torch.randn(pages, bs, H, D, device=device, generator=gen).to(torch.float16)
    v_pool = torch.randn(pages, bs, H, D, device=device, generator=gen).to(torch.float16)
    tables = torch.randperm(pages, device=device, generator=gen)[:B * 16].reshape(B, 16)
    tables = tables.to(torch.int32)
    lens = torch.tensor([5, 100, 17, 200], dtype=torch.int32, device=device)
    q = torch.empty(B, 1, H, D, device=device, dtype=torch.float16)
    kn = torch.empty(B, 1, H, D, device=device, dtype=torch.float16)
    vn = torch.empty_like(kn)
    pos = torch.empty(B, dtype=torch.int32, device=device)
    ones = torch.ones(B, dtype=torch.int32, device=device)
    errors = torch.full((3,), 7, dtype=torch.int32, device=device)

    def step():
        # the caller's error words: the append allocates nothing under capture
        store_kv(k_pool, v_pool, tables, kn, vn, pos, num_tokens=ones, check=False,
                 errors=errors)
        return paged_attention(q, k_pool, v_pool, tables, lens, block_size=bs)

    def fresh():
        for x in (q, kn, vn):
            x.copy_(torch.randn(x.shape, device=device, generator=gen).to(torch.float16))
        pos.copy_(lens)
        lens.add_(1)

    fresh()
    g, out = capture(step)
    for _ in range(4):
        fresh()
        kp0, vp0 = k_pool.clone(), v_pool.clone()
        g.replay()
        torch.cuda.synchronize()
        got, kp1, vp1 = out.clone(), k_pool.clone(), v_pool.clone()
        k_pool.copy_(kp0)
        v_pool.copy_(vp0)
        eager = step()
        torch.cuda.synchronize()
        assert torch.equal(k_pool, kp1) and torch.equal(v_pool, vp1)
        assert torch.equal(got, eager)
        assert errors.tolist() == [0, 0, 0]

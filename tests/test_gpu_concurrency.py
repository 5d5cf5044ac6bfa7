"""Concurrent calls from several host threads (the reference's stress tests,
tests/stress/test_concurrency.py:150-345, run attention from a thread pool
behind a mutex; here no caller-side lock is needed). Every result must equal
the same call made alone, bit for bit, whether the threads share torch's
default stream or each launches on its own stream.
"""

import concurrent.futures

import numpy as np
import pytest
import torch

from mlx_primitives.attention import flash_attention, sliding_window_attention
from mlx_primitives.cache import paged_attention

pytestmark = pytest.mark.gpu


def inputs(seed, device):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(1, 256, 8, 64, generator=g).to(torch.bfloat16).to(device)
               for _ in range(3))
    return q, k, v


def paged_inputs(seed, device):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(3, 1, 8, 64, generator=g).to(torch.float16).to(device)
    kp = torch.randn(40, 16, 8, 64, generator=g).to(torch.float16).to(device)
    vp = torch.randn(40, 16, 8, 64, generator=g).to(torch.float16).to(device)
    tables = torch.randperm(40, generator=g)[:39].reshape(3, 13).to(torch.int32).to(device)
    lens = torch.tensor([200, 7, 150], dtype=torch.int32, device=device)
    return q, kp, vp, tables, lens


def job(kind, seed, device, own_stream):
    stream = torch.cuda.Stream(device) if own_stream else None
    ctx = torch.cuda.stream(stream) if own_stream else torch.cuda.StreamContext(None)
    with ctx:
        if kind == "flash":
            out = flash_attention(*inputs(seed, device), causal=True)
        elif kind == "window":
            out = sliding_window_attention(*inputs(seed, device), window_size=17, causal=True)
        elif kind == "grad":
            q, k, v = (x.requires_grad_(True) for x in inputs(seed, device))
            flash_attention(q, k, v, causal=True).float().square().sum().backward()
            out = torch.cat([q.grad, k.grad, v.grad])
        else:
            out = paged_attention(*paged_inputs(seed, device))
        if own_stream:
            stream.synchronize()
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("own_stream", [False, True])
def test_threads_match_sequential(device, own_stream):
    tasks = [(kind, seed) for seed in range(4) for kind in ("flash", "window", "grad", "paged")]
    alone = {t: job(*t, device, False) for t in tasks}
    for _ in range(3):
        with concurrent.futures.ThreadPoolExecutor(max_workers=8) as ex:
            futs = {t: ex.submit(job, *t, device, own_stream) for t in tasks}
            for t, f in futs.items():
                got = f.result()
                assert torch.equal(got, alone[t]) or (
                    t[0] == "paged" and np.array_equal(got.numpy(), alone[t].numpy(),
                                                       equal_nan=True)), t

"""GPU parity of paged-KV decode (HIP kernel through the C ABI) against the
CPU oracle (oracle/paged.py) on identical inputs.

Tolerance: float32 rtol 1e-4 / atol 1e-5; float16 / bfloat16 max-abs <= 2e-2
against the float64 oracle run on the cast inputs.
"""

import math

import numpy as np
import pytest
import torch

from mlx_primitives.cache import create_block_table_from_lengths, get_alibi_slopes, paged_attention
from oracle import paged as op
import workloads as wl

pytestmark = pytest.mark.gpu


def check(out, ref, dtype):
    got = out.double().cpu().numpy()
    assert got.shape == ref.shape
    if dtype == torch.float32:
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
    else:
        err = np.nanmax(np.abs(got - ref))
        assert err <= 2e-2, f"max abs err {err}"


def run_case(device, dtype, lens, tables, num_blocks, bs, H, D, alibi=False, seed=0,
             oracle_tables=None):
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    q = torch.randn(B, 1, H, D, generator=g).to(dtype)
    kp = torch.randn(num_blocks, bs, H, D, generator=g).to(dtype)
    vp = torch.randn(num_blocks, bs, H, D, generator=g).to(dtype)
    tables = torch.as_tensor(np.asarray(tables), dtype=torch.int32)
    lens_t = torch.as_tensor(lens, dtype=torch.int32)
    slopes = get_alibi_slopes(H) if alibi else None
    out = paged_attention(q.to(device), kp.to(device), vp.to(device), tables.to(device),
                          lens_t.to(device), block_size=bs,
                          alibi_slopes=slopes.to(device) if alibi else None)
    assert out.shape == (B, 1, H, D) and out.dtype == dtype
    ref_tables = tables.numpy() if oracle_tables is None else np.asarray(oracle_tables, np.int32)
    ref = op.paged_attention(q.double().numpy(), kp.double().numpy(), vp.double().numpy(),
                             ref_tables, lens_t.numpy(), block_size=bs,
                             alibi_slopes=slopes.numpy() if alibi else None)
    return out, ref


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("alibi", [False, True])
def test_reference_tables(device, dtype, alibi):
    # tests/cache/test_paged_attention.py:164-197
    out, ref = run_case(device, dtype, [16, 32, 48, 25],
                        [[0, -1, -1], [1, 2, -1], [3, 4, 5], [6, 7, -1]], 20, 16, 8, 64, alibi)
    check(out, ref, dtype)


@pytest.mark.parametrize("lens,tables,nb", [
    ([30], [[0, 1]], 10),              # test_paged_attention.py:132-162
    ([32, 48], [[0, 1, -1], [2, 3, 4]], 10),   # 199-230
    ([1], [[0]], 5),                   # 232-259
])
def test_reference_small_cases(device, lens, tables, nb):
    out, ref = run_case(device, torch.float32, lens, tables, nb, 16, 8, 64)
    check(out, ref, torch.float32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bs", [1, 8, 16, 24, 32, 48, 128])
@pytest.mark.parametrize("D", [32, 64, 128, 256])
def test_random_tables(device, dtype, bs, D):
    rng = np.random.default_rng(bs * 1000 + D)
    B, H = 5, 6  # three workgroups of 2 heads; not a multiple of the grouped launch's 4
    lens = rng.integers(1, 2000, B)
    pages = (lens + bs - 1) // bs
    nb = int(pages.sum()) + 3
    perm = rng.permutation(nb)
    width = int(pages.max()) + 2
    tables = np.full((B, width), -1, np.int32)
    off = 0
    for b in range(B):
        tables[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    out, ref = run_case(device, dtype, lens.tolist(), tables, nb, bs, H, D, alibi=(bs == 16))
    check(out, ref, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("H", [1, 5, 7])
@pytest.mark.parametrize("alibi", [False, True])
def test_odd_head_counts(device, dtype, H, alibi):
    # The decode launch runs 2 query heads per workgroup without grouped heads
    # (4 with them): an odd H leaves the last workgroup one wave with no head.
    rng = np.random.default_rng(40 + H)
    lens = [700, 1, 1500]
    nb = sum((n + 15) // 16 for n in lens) + 2
    perm = rng.permutation(nb)
    tables = np.full((3, 100), -1, np.int32)
    off = 0
    for b, n in enumerate(lens):
        p = (n + 15) // 16
        tables[b, :p] = perm[off:off + p]
        off += p
    out, ref = run_case(device, dtype, lens, tables, nb, 16, H, 64, alibi=alibi, seed=H)
    check(out, ref, dtype)


@pytest.mark.parametrize("dtype,D", [(torch.float16, 80), (torch.bfloat16, 96),
                                     (torch.bfloat16, 48), (torch.float32, 100),
                                     (torch.float32, 20), (torch.float16, 8),
                                     (torch.bfloat16, 100), (torch.float16, 30),
                                     (torch.bfloat16, 200), (torch.float32, 136),
                                     (torch.float16, 150)])
def test_unpadded_head_dims(device, dtype, D):
    # Head dims that are multiples of the 16-byte vector are read in place by
    # the decode kernel; others copy only the referenced pages, padded.
    out, ref = run_case(device, dtype, [40, 300, 17], [[3, 0, 5, -1, -1, -1, -1, -1, -1, -1, -1,
                                                        -1, -1, -1, -1, -1, -1, -1, -1, -1],
                                                       list(range(6, 25)) + [-1],
                                                       [1, 2] + [-1] * 18], 26, 16, 3, D,
                        alibi=True, seed=D)
    check(out, ref, dtype)


def test_decode_reads_pools_in_place(device):
    # Decode over pools of a head dim the kernel does not instantiate (80 ->
    # the 128 kernel) allocates nothing of the pools' size.
    g = torch.Generator().manual_seed(3)
    nb, bs, H, D = 4096, 16, 8, 80
    kp = torch.randn(nb, bs, H, D, generator=g).to(torch.float16).to(device)
    vp = torch.randn(nb, bs, H, D, generator=g).to(torch.float16).to(device)
    q = torch.randn(2, 1, H, D, generator=g).to(torch.float16).to(device)
    tables = torch.arange(2 * 64, dtype=torch.int32, device=device).reshape(2, 64)
    lens = torch.tensor([1000, 64 * 16], dtype=torch.int32, device=device)
    paged_attention(q, kp, vp, tables, lens, block_size=bs)  # warm the allocator
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(device)
    base = torch.cuda.memory_allocated(device)
    out = paged_attention(q, kp, vp, tables, lens, block_size=bs)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated(device) - base
    assert peak < kp.numel() * kp.element_size() // 16, peak
    ref = op.paged_attention(q.double().cpu().numpy(), kp.double().cpu().numpy(),
                             vp.double().cpu().numpy(), tables.cpu().numpy(),
                             lens.cpu().numpy(), block_size=bs)
    check(out, ref, torch.float16)


@pytest.mark.parametrize("D", [80, 30])
def test_prefill_unpadded_head_dims(device, D):
    # Prefill with a head dim the kernels do not instantiate: only the
    # referenced pages are copied (padded); page 2 is referenced by neither row.
    g = torch.Generator().manual_seed(D)
    nb, bs, H = 6, 16, 2
    q = torch.randn(2, 20, H, D, generator=g).to(torch.bfloat16)
    kp = torch.randn(nb, bs, H, D, generator=g).to(torch.bfloat16)
    vp = torch.randn(nb, bs, H, D, generator=g).to(torch.bfloat16)
    tables = torch.tensor([[5, 0, -1], [3, 1, 4]], dtype=torch.int32)
    lens = torch.tensor([25, 40], dtype=torch.int32)
    out = paged_attention(q.to(device), kp.to(device), vp.to(device), tables.to(device),
                          lens.to(device), block_size=bs)
    ref = op.paged_attention(q.double().numpy(), kp.double().numpy(), vp.double().numpy(),
                             tables.numpy(), lens.numpy(), block_size=bs)
    check(out, ref, torch.bfloat16)


def test_invalid_pages_are_masked(device):
    # A -1 page inside the context is masked (reference semantics); an id past
    # the pool is masked the same way and never dereferenced (the reference
    # would gather out of bounds), so the oracle sees it as -1.
    out, ref = run_case(device, torch.float32, [40, 40], [[0, -1, 2], [1, 99, 3]], 4, 16, 4, 64,
                        oracle_tables=[[0, -1, 2], [1, -1, 3]])
    check(out, ref, torch.float32)


def test_empty_context_is_nan(device):
    out, ref = run_case(device, torch.float32, [0, 20], [[0, 1], [2, 3]], 4, 16, 4, 64)
    got = out.cpu().numpy()
    assert np.isnan(got[0]).all() and np.isnan(ref[0]).all()
    np.testing.assert_allclose(got[1], ref[1], rtol=1e-4, atol=1e-5)


def test_block_table_helper_feeds_kernel(device):
    lens = torch.tensor([100, 5, 33], dtype=torch.int32)
    tables = create_block_table_from_lengths(lens, 16)
    nb = int(((lens + 15) // 16).sum())
    out, ref = run_case(device, torch.float16, lens.tolist(), tables.numpy(), nb, 16, 4, 128)
    check(out, ref, torch.float16)


def test_deterministic(device):
    out1, _ = run_case(device, torch.float16, [3000, 700], [[i for i in range(188)], [188 + i for i in range(44)] + [-1] * 144], 232, 16, 8, 128)
    out2, _ = run_case(device, torch.float16, [3000, 700], [[i for i in range(188)], [188 + i for i in range(44)] + [-1] * 144], 232, 16, 8, 128)
    assert torch.equal(out1, out2)


def test_config4_paged_decode_full(device):
    cfg = wl.CONFIGS["paged_decode_fp16"]
    inp = wl.make_paged(cfg, device="cpu")
    out = paged_attention(inp.q.to(device), inp.k_pool.to(device), inp.v_pool.to(device),
                          inp.block_tables.to(device), inp.context_lens.to(device),
                          block_size=inp.block_size)
    # Oracle in float32 on the cast inputs for all 64 sequences.
    ref = op.paged_attention(inp.q.float().numpy(), inp.k_pool.float().numpy(),
                             inp.v_pool.float().numpy(), inp.block_tables.numpy(),
                             inp.context_lens.numpy(), block_size=inp.block_size)
    err = np.abs(out.double().cpu().numpy() - ref).max()
    assert err <= 2e-2, err

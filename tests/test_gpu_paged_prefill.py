"""GPU parity of paged-KV prefill (seq_q > 1; HIP flash kernel with block-table
indirection, through the C ABI) against the CPU oracle (oracle/paged.py).

Tolerance: float32 rtol 1e-4 / atol 1e-5; float16 / bfloat16 max-abs <= 2e-2
against the float64 oracle run on the cast inputs. NaN rows (queries with no
valid key) must be NaN in both.
"""

import numpy as np
import pytest
import torch

from mlx_primitives.cache import get_alibi_slopes, paged_attention
from oracle import paged as op

pytestmark = pytest.mark.gpu


def check(out, ref, dtype):
    got = out.double().cpu().numpy()
    assert got.shape == ref.shape
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    if dtype == torch.float32:
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
    else:
        err = np.nanmax(np.abs(got - ref)) if np.isfinite(ref).any() else 0.0
        assert err <= 2e-2, f"max abs err {err}"


def run_case(device, dtype, Sq, lens, tables, num_blocks, bs, H, D, causal=True, alibi=False,
             seed=0, oracle_tables=None, q_layout="bshd"):
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    if q_layout == "bhsd":  # a (B, Sq, H, D) view of a head-major tensor
        q = torch.randn(B, H, Sq, D, generator=g).to(dtype).transpose(1, 2)
    else:
        q = torch.randn(B, Sq, H, D, generator=g).to(dtype)
    kp = torch.randn(num_blocks, bs, H, D, generator=g).to(dtype)
    vp = torch.randn(num_blocks, bs, H, D, generator=g).to(dtype)
    tables = torch.as_tensor(np.asarray(tables), dtype=torch.int32)
    lens_t = torch.as_tensor(lens, dtype=torch.int32)
    slopes = get_alibi_slopes(H) if alibi else None
    qd = q.to(device) if q_layout == "bshd" else q.transpose(1, 2).contiguous().to(device).transpose(1, 2)
    out = paged_attention(qd, kp.to(device), vp.to(device), tables.to(device), lens_t.to(device),
                          block_size=bs, causal=causal,
                          alibi_slopes=slopes.to(device) if alibi else None)
    assert out.shape == (B, Sq, H, D) and out.dtype == dtype
    ref_tables = tables.numpy() if oracle_tables is None else np.asarray(oracle_tables, np.int32)
    ref = op.paged_attention(q.double().numpy(), kp.double().numpy(), vp.double().numpy(),
                             ref_tables, lens_t.numpy(), block_size=bs, causal=causal,
                             alibi_slopes=slopes.numpy() if alibi else None)
    return out, ref


# tests/cache/test_paged_attention.py:493-620 (shapes, tables, lengths, causal flag)
@pytest.mark.parametrize("Sq,lens,tables,nb,causal", [
    (10, [10], [[0]], 5, True),                       # 493-521
    (20, [20, 20], [[0, 1], [2, 3]], 10, True),       # 523-553
    (50, [50], [[0, 1, 2, 3]], 10, True),             # 555-585
    (16, [16], [[0]], 5, False),                      # 587-615
    (25, [25, 25], [[0, 1], [2, 3]], 10, True),       # 617-630 (output shape)
])
def test_reference_cases(device, Sq, lens, tables, nb, causal):
    out, ref = run_case(device, torch.float32, Sq, lens, tables, nb, 16, 8, 64, causal=causal)
    check(out, ref, torch.float32)


def random_tables(rng, lens, bs, extra=3, holes=True):
    pages = [(int(n) + bs - 1) // bs for n in lens]
    nb = sum(pages) + extra
    perm = rng.permutation(nb)
    width = max(pages) + 2
    tables = np.full((len(lens), width), -1, np.int32)
    off = 0
    for b, n in enumerate(pages):
        tables[b, :n] = perm[off:off + n]
        off += n
    if holes and pages[0] > 2:
        tables[0, 1] = -1  # a missing page inside the context is masked
    return tables, nb


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [32, 64, 128, 256, 200])
@pytest.mark.parametrize("causal", [True, False])
def test_random_tables(device, dtype, D, causal):
    rng = np.random.default_rng(D * 7 + int(causal))
    Sq, H, bs = 150, 5, 16
    lens = [400, 150, 37]  # context longer than, equal to and shorter than the queries
    tables, nb = random_tables(rng, lens, bs)
    out, ref = run_case(device, dtype, Sq, lens, tables, nb, bs, H, D, causal=causal,
                        alibi=(D == 64), seed=D)
    check(out, ref, dtype)


@pytest.mark.parametrize("bs", [1, 8, 24, 48, 128])
def test_block_sizes(device, bs):
    # power-of-two and other page sizes; pages smaller and larger than a kv tile
    rng = np.random.default_rng(bs)
    lens = [333, 70]
    tables, nb = random_tables(rng, lens, bs)
    out, ref = run_case(device, torch.bfloat16, 90, lens, tables, nb, bs, 4, 128, seed=bs)
    check(out, ref, torch.bfloat16)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 64),
                                     (torch.float32, 128), (torch.bfloat16, 256),
                                     (torch.float32, 256)])
def test_split_kv_long_context(device, dtype, D):
    # few query tiles over a long table: the kv range is split across workgroups
    # and merged (the workspace path)
    rng = np.random.default_rng(11)
    lens = [6000]
    tables, nb = random_tables(rng, lens, 16)
    out, ref = run_case(device, dtype, 70, lens, tables, nb, 16, 4, D, causal=False, alibi=True)
    check(out, ref, dtype)


def test_causal_long_context_alibi_f32(device):
    # causal rows see keys <= their own position inside a long table; ALiBi
    # bias accuracy in float32 on both sides of the split
    rng = np.random.default_rng(12)
    lens = [3000, 250]
    tables, nb = random_tables(rng, lens, 16)
    out, ref = run_case(device, torch.float32, 300, lens, tables, nb, 16, 4, 128, causal=True,
                        alibi=True)
    check(out, ref, torch.float32)


@pytest.mark.parametrize("dtype,D", [(torch.float32, 64), (torch.bfloat16, 128),
                                     (torch.float16, 64)])
def test_invalid_page_ids_masked(device, dtype, D):
    # ids past the pool are masked like -1 and never dereferenced
    out, ref = run_case(device, dtype, 40, [40, 40], [[0, -1, 2], [1, 99, 3]], 4, 16, 4,
                        D, causal=False, oracle_tables=[[0, -1, 2], [1, -1, 3]])
    check(out, ref, dtype)


@pytest.mark.parametrize("bs,D", [(4, 128), (8, 64), (4, 64), (256, 64), (32, 128)])
@pytest.mark.parametrize("holes", [False, True])
def test_block_sizes_wide_tiles(device, bs, D, holes):
    # 128-key tiles read page ids from the table (power-of-two pages of at
    # least 4 rows at D = 128, 8 at D = 64); other page sizes take the 64-key
    # kernel. Tables with and without missing pages inside the context.
    rng = np.random.default_rng(bs * D + int(holes))
    lens = [700, 129, 1]
    tables, nb = random_tables(rng, lens, bs, holes=holes)
    out, ref = run_case(device, torch.float16, 200, lens, tables, nb, bs, 3, D, seed=bs + D)
    check(out, ref, torch.float16)


def test_empty_rows_are_nan(device):
    # sequence 0 has no context; sequence 1's first page is missing, so its
    # first 16 causal query rows see no key
    out, ref = run_case(device, torch.bfloat16, 20, [0, 20], [[0, 1], [-1, 3]], 4, 16, 4, 128)
    got = out.float().cpu().numpy()
    assert np.isnan(got[0]).all() and np.isnan(got[1, :16]).all()
    assert np.isfinite(got[1, 16:]).all()
    check(out, ref, torch.bfloat16)


def test_empty_pool_is_nan(device):
    q = torch.randn(2, 5, 4, 64, device=device, dtype=torch.float16)
    pool = torch.empty(0, 16, 4, 64, device=device, dtype=torch.float16)
    tables = torch.full((2, 3), -1, dtype=torch.int32, device=device)
    lens = torch.tensor([10, 0], dtype=torch.int32, device=device)
    out = paged_attention(q, pool, pool, tables, lens, block_size=16)
    assert torch.isnan(out).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_head_major_query_view(device, dtype):
    rng = np.random.default_rng(3)
    lens = [300, 129]
    tables, nb = random_tables(rng, lens, 16)
    out, ref = run_case(device, dtype, 129, lens, tables, nb, 16, 6, 128, q_layout="bhsd")
    check(out, ref, dtype)


def test_page_permutation_invariance(device):
    # Size-independent property at a serving shape: permuting the pool's pages
    # and the tables together leaves the result bit-identical.
    g = torch.Generator().manual_seed(9)
    B, Sq, H, D, bs = 2, 1024, 16, 128, 16
    ctx = [2048, 1500]
    pages = [(n + bs - 1) // bs for n in ctx]
    nb = sum(pages)
    q = torch.randn(B, Sq, H, D, generator=g).to(torch.bfloat16).to(device)
    kp = torch.randn(nb, bs, H, D, generator=g).to(torch.bfloat16).to(device)
    vp = torch.randn(nb, bs, H, D, generator=g).to(torch.bfloat16).to(device)
    width = max(pages)
    ident = torch.full((B, width), -1, dtype=torch.int32)
    ident[0, :pages[0]] = torch.arange(pages[0])
    ident[1, :pages[1]] = pages[0] + torch.arange(pages[1])
    perm = torch.randperm(nb, generator=g)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(nb)
    # page p of the identity layout lives at slot inv[p] of the permuted pool
    permuted = torch.where(ident >= 0, inv[ident.clamp(min=0).long()].int(), ident)
    lens = torch.tensor(ctx, dtype=torch.int32, device=device)
    a = paged_attention(q, kp, vp, ident.to(device), lens, block_size=bs)
    b = paged_attention(q, kp[perm.to(device)], vp[perm.to(device)], permuted.to(device), lens,
                        block_size=bs)
    torch.cuda.synchronize()
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b)


def test_deterministic(device):
    rng = np.random.default_rng(5)
    lens = [3000, 700]
    tables, nb = random_tables(rng, lens, 16)
    o1, _ = run_case(device, torch.float16, 64, lens, tables, nb, 16, 8, 128, causal=False)
    o2, _ = run_case(device, torch.float16, 64, lens, tables, nb, 16, 8, 128, causal=False)
    assert torch.equal(o1, o2)


# Pools of 4 GiB and more: the 16-bit kernels read pages through 64-bit
# addresses (the 32-bit buffer offsets end below 4 GiB). The pools are left
# uninitialised except for the referenced pages, which sit both below and above
# the 4 GiB mark; the oracle runs on those pages alone (a compact pool with the
# table renumbered), so unreferenced memory cannot reach the result.
@pytest.mark.parametrize("dtype,D,H,H_kv,bs,alibi,Sq", [
    (torch.bfloat16, 128, 8, 8, 16, False, 300),   # 128-key tiles, page ids per instruction
    (torch.float16, 128, 8, 4, 16, True, 300),     # 64-key tiles, page-table slice (ALiBi)
    (torch.bfloat16, 128, 4, 4, 24, False, 200),   # page size not a power of two
    (torch.bfloat16, 64, 8, 8, 16, False, 300),
    (torch.float16, 32, 8, 8, 16, False, 200),     # register-staged tiles
    (torch.bfloat16, 256, 4, 2, 16, False, 150),   # head dim 256 (register-staged)
    (torch.float16, 128, 32, 8, 16, False, 1),     # decode: grouped-query MFMA kernel
    (torch.bfloat16, 128, 16, 4, 24, True, 1),     # the same, page size 24, ALiBi
    (torch.bfloat16, 64, 8, 8, 16, False, 1),      # decode: per-head kernel
])
def test_pool_above_4gib(device, dtype, D, H, H_kv, bs, alibi, Sq):
    rng = np.random.default_rng(D + bs + H_kv)
    block_bytes = bs * H_kv * D * 2
    nb = (4 << 30) // block_bytes + 4096  # 4 GiB + 4096 pages
    lens = [700, Sq, 1000]
    pages = [(n + bs - 1) // bs for n in lens]
    # referenced pages: most of them past 4 GiB, some below, in random order
    high = rng.choice(np.arange((4 << 30) // block_bytes, nb), sum(pages) - 6, replace=False)
    low = rng.choice(np.arange(0, 1000), 6, replace=False)
    ids = rng.permutation(np.concatenate([high, low]))
    width = max(pages) + 1
    tables = np.full((3, width), -1, np.int32)
    off = 0
    for b, n in enumerate(pages):
        tables[b, :n] = ids[off:off + n]
        off += n
    tables[0, 3] = -1  # a missing page inside the context
    g = torch.Generator().manual_seed(int(nb))
    q = torch.randn(3, Sq, H, D, generator=g).to(dtype)
    kc = torch.randn(len(ids), bs, H_kv, D, generator=g).to(dtype)
    vc = torch.randn(len(ids), bs, H_kv, D, generator=g).to(dtype)
    kp = torch.empty((nb, bs, H_kv, D), dtype=dtype, device=device)
    vp = torch.empty((nb, bs, H_kv, D), dtype=dtype, device=device)
    assert kp.numel() * 2 >= 4 << 30
    idx = torch.as_tensor(ids, dtype=torch.long).to(device)
    kp[idx] = kc.to(device)
    vp[idx] = vc.to(device)
    slopes = get_alibi_slopes(H) if alibi else None
    lens_t = torch.as_tensor(lens, dtype=torch.int32)
    print(f"pool {kp.numel() * 2 / 2**30:.2f} GiB, {dtype}, D={D}, bs={bs}, Sq={Sq}", flush=True)
    out = paged_attention(q.to(device), kp, vp, torch.as_tensor(tables).to(device),
                          lens_t.to(device), block_size=bs, causal=True,
                          alibi_slopes=slopes.to(device) if alibi else None,
                          enable_gqa=H != H_kv)
    torch.cuda.synchronize()
    del kp, vp
    # the oracle on the referenced pages: compact pool, renumbered table
    where = {int(p): i for i, p in enumerate(ids)}
    ctab = np.vectorize(lambda p: where.get(int(p), -1))(tables).astype(np.int32)
    ctab[tables < 0] = -1
    grp = H // H_kv
    ref = op.paged_attention(q.double().numpy(),
                             kc.repeat_interleave(grp, dim=2).double().numpy(),
                             vc.repeat_interleave(grp, dim=2).double().numpy(), ctab,
                             lens_t.numpy(), block_size=bs, causal=True,
                             alibi_slopes=slopes.numpy() if alibi else None)
    check(out, ref, dtype)

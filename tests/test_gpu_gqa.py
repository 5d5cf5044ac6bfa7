"""GPU checks of grouped-query attention (K/V with fewer heads than Q) on the
flash, paged-decode and paged-prefill kernels, through the C ABI.

Two bars: the float64 oracle on K/V whose heads are repeated to the query
heads (float32 rtol 1e-4 / atol 1e-5; 16-bit max-abs <= 2e-2), and bit
identity with the same kernel run on the expanded K/V (each query head reads
exactly the K/V head it would read after expansion).
"""

import math

import numpy as np
import pytest
import torch

from mlx_primitives.attention import flash_attention
from mlx_primitives.cache import paged_attention
from oracle import attention as oa
from oracle import paged as op

pytestmark = pytest.mark.gpu


def rnd(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype)


def check(out, ref, dtype):
    got = out.double().cpu().numpy()
    if dtype == torch.float32:
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
    else:
        err = float(np.nanmax(np.abs(got - ref)))
        assert err <= 2e-2, f"max abs err {err}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("layout", ["BSHD", "BHSD"])
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("H,H_kv", [(8, 1), (8, 2), (6, 3)])
def test_flash_gqa(device, dtype, layout, D, H, H_kv):
    B, S = 2, 300
    hax = 2 if layout == "BSHD" else 1
    qs = (B, S, H, D) if layout == "BSHD" else (B, H, S, D)
    ks = (B, S, H_kv, D) if layout == "BSHD" else (B, H_kv, S, D)
    q, k, v = rnd(qs, D + H, dtype), rnd(ks, D + H + 1, dtype), rnd(ks, D + H + 2, dtype)
    out = flash_attention(q.to(device), k.to(device), v.to(device), causal=True, layout=layout,
                          enable_gqa=True)
    g = H // H_kv
    ke, ve = k.repeat_interleave(g, dim=hax), v.repeat_interleave(g, dim=hax)
    same = flash_attention(q.to(device), ke.to(device), ve.to(device), causal=True,
                           layout=layout)
    torch.cuda.synchronize()
    assert torch.equal(out, same)
    ref = oa.flash_attention(q.double().numpy(), ke.double().numpy(), ve.double().numpy(),
                             1 / math.sqrt(D), True, layout=layout)
    check(out, ref, dtype)


def test_flash_gqa_headline_shape_identity(device):
    # the direct (DMA) kernel at a serving shape: 32 query heads over 8 K/V heads
    q = rnd((2, 32, 2048, 128), 1, torch.bfloat16).to(device)
    k = rnd((2, 8, 2048, 128), 2, torch.bfloat16).to(device)
    v = rnd((2, 8, 2048, 128), 3, torch.bfloat16).to(device)
    out = flash_attention(q, k, v, causal=True, layout="BHSD", enable_gqa=True)
    same = flash_attention(q, k.repeat_interleave(4, dim=1), v.repeat_interleave(4, dim=1),
                           causal=True, layout="BHSD")
    torch.cuda.synchronize()
    assert torch.equal(out, same)


def paged_inputs(dtype, B, Sq, H, H_kv, D, bs, lens, seed):
    rng = np.random.default_rng(seed)
    pages = [(n + bs - 1) // bs for n in lens]
    nb = sum(pages) + 2
    perm = rng.permutation(nb)
    tables = np.full((B, max(pages)), -1, np.int32)
    off = 0
    for b, n in enumerate(pages):
        tables[b, :n] = perm[off:off + n]
        off += n
    q = rnd((B, Sq, H, D), seed, dtype)
    kp = rnd((nb, bs, H_kv, D), seed + 1, dtype)
    vp = rnd((nb, bs, H_kv, D), seed + 2, dtype)
    return q, kp, vp, torch.from_numpy(tables), torch.tensor(lens, dtype=torch.int32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Sq", [1, 77])
@pytest.mark.parametrize("H,H_kv,D", [(32, 8, 128), (8, 1, 64), (12, 4, 128), (8, 2, 256)])
def test_paged_gqa(device, dtype, Sq, H, H_kv, D):
    lens = [700, 33, 400]
    q, kp, vp, tables, lens_t = paged_inputs(dtype, 3, Sq, H, H_kv, D, 16, lens, H + D + Sq)
    d = lambda x: x.to(device)
    out = paged_attention(d(q), d(kp), d(vp), d(tables), d(lens_t), causal=True,
                          enable_gqa=True)
    g = H // H_kv
    kpe, vpe = kp.repeat_interleave(g, dim=2), vp.repeat_interleave(g, dim=2)
    same = paged_attention(d(q), d(kpe), d(vpe), d(tables), d(lens_t), causal=True)
    torch.cuda.synchronize()
    ref = op.paged_attention(q.double().numpy(), kpe.double().numpy(), vpe.double().numpy(),
                             tables.numpy(), lens_t.numpy(), block_size=16, causal=True)
    if Sq == 1 and dtype != torch.float32 and D == 128 and 2 <= g <= 16:
        # 16-bit grouped decode at D = 128 runs the MFMA kernel (each K/V row
        # scored against the whole group); the expanded heads take the
        # per-head kernel: both against the oracle
        check(same, ref, dtype)
    else:
        assert torch.equal(out, same)
    check(out, ref, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("H,H_kv,D", [(16, 8, 128), (16, 4, 64), (64, 8, 128), (8, 1, 32),
                                      (24, 8, 128)])
def test_gqa_decode_alibi_ragged(device, dtype, H, H_kv, D):
    # groups 2, 3, 4, 8 with ALiBi, ragged contexts incl. a missing page and an
    # empty sequence (NaN row)
    from mlx_primitives.cache import get_alibi_slopes

    lens = [1000, 1, 0, 517]
    q, kp, vp, tables, lens_t = paged_inputs(dtype, 4, 1, H, H_kv, D, 16, lens, H + D)
    tables[3, 5] = -1
    d = lambda x: x.to(device)
    slopes = get_alibi_slopes(H)
    out = paged_attention(d(q), d(kp), d(vp), d(tables), d(lens_t), alibi_slopes=d(slopes),
                          enable_gqa=True)
    g = H // H_kv
    ref = op.paged_attention(q.double().numpy(), kp.repeat_interleave(g, dim=2).double().numpy(),
                             vp.repeat_interleave(g, dim=2).double().numpy(), tables.numpy(),
                             lens_t.numpy(), block_size=16, alibi_slopes=slopes.double().numpy())
    got = out.double().cpu().numpy()
    assert np.isnan(got[2]).all() and np.isnan(ref[2]).all()
    check(out[[0, 1, 3]], ref[[0, 1, 3]], dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("H,H_kv,bs", [(16, 1, 16), (32, 2, 1), (48, 4, 8), (20, 10, 32),
                                       (34, 2, 64), (12, 3, 24), (16, 2, 48)])
def test_gqa_mfma_decode_groups_and_pages(device, dtype, H, H_kv, bs):
    # the MFMA decode kernel: groups 16, 16, 12, 2, 17 (> 16: per-head
    # kernel), 4 and 8, page sizes 1 .. 64 (24 and 48: not powers of two),
    # contexts ending mid-tile and mid-page, several partitions, a missing page
    lens = [1537, 31, 512, 2049]
    q, kp, vp, tables, lens_t = paged_inputs(dtype, 4, 1, H, H_kv, 128, bs, lens, H + bs)
    tables[0, 3] = -1
    d = lambda x: x.to(device)
    out = paged_attention(d(q), d(kp), d(vp), d(tables), d(lens_t), block_size=bs,
                          enable_gqa=True)
    g = H // H_kv
    ref = op.paged_attention(q.double().numpy(), kp.repeat_interleave(g, dim=2).double().numpy(),
                             vp.repeat_interleave(g, dim=2).double().numpy(), tables.numpy(),
                             lens_t.numpy(), block_size=bs)
    check(out, ref, dtype)

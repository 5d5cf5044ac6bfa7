"""GPU parity of the KV-cache page writes (HIP scatter kernel through the C ABI)
against the CPU oracle (oracle/kv_cache.py). Page writes are copies: the
pools must match the oracle's bit for bit.
"""

import math

import numpy as np
import pytest
import torch

from mlx_primitives.cache import paged_attention, set_block_data, store_kv
from oracle import kv_cache as ok
from oracle import paged as op

pytestmark = pytest.mark.gpu


def make(rng, shape, dtype):
    return torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(dtype)


def as_np(t):
    # bit patterns, so that the comparison is exact for every dtype
    return t.cpu().view(torch.int32 if t.dtype == torch.float32 else torch.int16).numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_ragged_append_matches_oracle(device, dtype, D):
    rng = np.random.default_rng(D)
    B, T, H, bs, nb = 4, 37, 3, 16, 40
    kp = make(rng, (nb, bs, H, D), dtype); vp = make(rng, (nb, bs, H, D), dtype)
    k = make(rng, (B, T, H, D), dtype); v = make(rng, (B, T, H, D), dtype)
    perm = rng.permutation(nb)
    tables = perm[:B * 8].reshape(B, 8).astype(np.int32)
    starts = [0, 13, 100, 31]          # page-aligned, mid-page, late in the table
    counts = [37, 1, 20, 0]            # full, decode-style, partial, nothing
    kd, vd = kp.to(device), vp.to(device)
    store_kv(kd, vd, torch.from_numpy(tables).to(device), k.to(device), v.to(device),
             torch.tensor(starts, dtype=torch.int32), torch.tensor(counts, dtype=torch.int32))
    kr, vr = kp.clone(), vp.clone()
    ok.kv_append(kr.numpy() if dtype == torch.float32 else kr.view(torch.int16).numpy(),
                 vr.numpy() if dtype == torch.float32 else vr.view(torch.int16).numpy(),
                 tables,
                 k.numpy() if dtype == torch.float32 else k.view(torch.int16).numpy(),
                 v.numpy() if dtype == torch.float32 else v.view(torch.int16).numpy(),
                 starts, counts)
    np.testing.assert_array_equal(as_np(kd), as_np(kr))
    np.testing.assert_array_equal(as_np(vd), as_np(vr))


def test_single_sequence_form_and_strided_input(device):
    # (T, H, D) input as KVCache._store_kv takes it, sliced out of a wider tensor
    rng = np.random.default_rng(1)
    H, D, bs, nb = 4, 64, 16, 6
    wide = make(rng, (21, H, 2 * D), torch.bfloat16).to(device)
    k, v = wide[..., :D], wide[..., D:]
    assert not k.is_contiguous()
    kp = torch.zeros(nb, bs, H, D, dtype=torch.bfloat16, device=device); vp = torch.zeros_like(kp)
    table = torch.tensor([5, 2, 0], dtype=torch.int32, device=device)
    store_kv(kp, vp, table, k, v, 9)
    pos = torch.arange(9, 30)
    pages = table.cpu()[pos // bs].long()
    assert torch.equal(kp.cpu()[pages, pos % bs], k.cpu())
    assert torch.equal(vp.cpu()[pages, pos % bs], v.cpu())
    untouched = torch.ones(nb, bs, dtype=torch.bool)
    untouched[pages, pos % bs] = False
    assert not kp.cpu()[untouched].any()


def test_set_block_data_kat(device):
    # tests/cache/test_block_allocator.py:97-119
    rng = np.random.default_rng(2)
    kp = torch.zeros(10, 16, 8, 64, dtype=torch.float16, device=device); vp = torch.zeros_like(kp)
    k = make(rng, (8, 8, 64), torch.float16).to(device); v = make(rng, (8, 8, 64), torch.float16).to(device)
    set_block_data(kp, vp, 3, k, v, start_pos=0, length=8)
    torch.cuda.synchronize()
    assert torch.equal(kp[3, :8], k) and torch.equal(vp[3, :8], v)
    assert not kp[3, 8:].any() and not kp[:3].any() and not kp[4:].any()


def test_errors_raise_like_reference(device):
    kp = torch.zeros(4, 4, 1, 8, device=device); vp = torch.zeros_like(kp)
    x = torch.ones(1, 3, 1, 8, device=device)
    tab = torch.tensor([[0, 1]], dtype=torch.int32, device=device)
    with pytest.raises(ValueError, match="write_start"):
        store_kv(kp, vp, tab, x, x, -1)
    with pytest.raises(RuntimeError, match="Block index"):
        store_kv(kp, vp, tab, x, x, 6)
    with pytest.raises(ValueError, match="block_id"):
        store_kv(kp, vp, torch.tensor([[0, 9]], dtype=torch.int32, device=device), x, x, 3)
    # without the check nothing waits; the flags say what happened and the
    # tokens that could be placed are written (positions 6, 7 -> page 1)
    kp.zero_()
    flags = store_kv(kp, vp, tab, 2 * x, x, 6, check=False)
    assert flags.tolist() == [0, 1, 0]
    assert (kp[1, 2:] == 2).all() and not kp[0].any()


def test_append_then_decode_and_prefill(device):
    # The caller's flow: write a prompt into pages, attend to it (prefill),
    # append one token per step, attend again (decode). Checked against the
    # oracle on a dense copy of what was written.
    rng = np.random.default_rng(4)
    B, H, D, bs, nb, P = 2, 4, 128, 16, 24, 40
    kp = torch.zeros(nb, bs, H, D, dtype=torch.bfloat16, device=device); vp = torch.zeros_like(kp)
    tables = torch.from_numpy(rng.permutation(nb)[:B * 6].reshape(B, 6).astype(np.int32)).to(device)
    k = make(rng, (B, P + 3, H, D), torch.bfloat16).to(device)
    v = make(rng, (B, P + 3, H, D), torch.bfloat16).to(device)
    q = make(rng, (B, P, H, D), torch.bfloat16).to(device)
    store_kv(kp, vp, tables, k[:, :P], v[:, :P], 0)
    lens = torch.full((B,), P, dtype=torch.int32, device=device)
    out = paged_attention(q, kp, vp, tables, lens, block_size=bs, causal=True)
    ref = op.paged_attention(q.double().cpu().numpy(), kp.double().cpu().numpy(),
                             vp.double().cpu().numpy(), tables.cpu().numpy(), lens.cpu().numpy(),
                             block_size=bs, causal=True)
    assert np.abs(out.double().cpu().numpy() - ref).max() <= 2e-2
    for step in range(3):
        pos = P + step
        store_kv(kp, vp, tables, k[:, pos:pos + 1], v[:, pos:pos + 1], pos)
        lens += 1
        qd = make(rng, (B, 1, H, D), torch.bfloat16).to(device)
        out = paged_attention(qd, kp, vp, tables, lens, block_size=bs)
        # dense reference over the appended tokens themselves
        kk = k[:, :pos + 1].double().cpu().numpy(); vv = v[:, :pos + 1].double().cpu().numpy()
        qq = qd.double().cpu().numpy()
        s = np.einsum("bhd,bthd->bht", qq[:, 0], kk) / math.sqrt(D)
        w = np.exp(s - s.max(-1, keepdims=True)); w /= w.sum(-1, keepdims=True)
        dense = np.einsum("bht,bthd->bhd", w, vv)[:, None]
        assert np.abs(out.double().cpu().numpy() - dense).max() <= 2e-2


def test_large_append_round_trip(device):
    # a serving-size prompt append (8 sequences x 4096 tokens x 32 heads x 128,
    # bf16: 2 x 256 MiB written) checked by reading every position back
    # through the tables
    g = torch.Generator(device="cpu").manual_seed(7)
    B, T, H, D, bs = 8, 4096, 32, 128, 16
    nb = B * T // bs + 64
    kp = torch.zeros(nb, bs, H, D, dtype=torch.bfloat16, device=device); vp = torch.zeros_like(kp)
    tables = torch.randperm(nb, generator=g)[:B * T // bs].reshape(B, T // bs).int().to(device)
    k = torch.randn(B, T, H, D, device=device).to(torch.bfloat16)
    v = torch.randn(B, T, H, D, device=device).to(torch.bfloat16)
    store_kv(kp, vp, tables, k, v, 0)
    back_k = kp[tables.long()].reshape(B, T, H, D)
    back_v = vp[tables.long()].reshape(B, T, H, D)
    assert torch.equal(back_k, k) and torch.equal(back_v, v)

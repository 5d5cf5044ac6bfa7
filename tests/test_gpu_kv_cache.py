"""The KV-cache producers on the GPU: BlockAllocator page data, KVCache
appends (the gfx950 append kernel) feeding paged attention, forks with
copy-on-write, rollback and batched appends.

The reference's serving stack is update -> get_kv_paged -> paged_attention
(tests/cache/test_paged_attention.py:339-395); here its output is checked
against the float64 oracle run on the same tokens laid out contiguously
(fp16: max-abs 2e-2), and every page write is checked bit for bit against the
tokens written.
"""

import numpy as np
import pytest
import torch

from mlx_primitives.cache import (
    BlockAllocator,
    BlockConfig,
    KVCache,
    KVCacheConfig,
    MultiLayerKVCache,
    paged_attention,
)
from oracle import attention as oa

pytestmark = pytest.mark.gpu


def rnd(shape, seed, dtype=torch.float16, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype).to(device)


def cache(device, num_layers=1, heads=8, dim=64, gb=0.1, bs=16, **kw):
    cfg = KVCacheConfig(num_heads=heads, head_dim=dim, num_layers=num_layers, max_memory_gb=gb,
                        block_size=bs, **kw)
    return KVCache(cfg, device=device)


def decode_ref(q, ks, vs):
    """Decode attention of q (B, 1, H, D) over each sequence's contiguous K/V."""
    out = []
    for b, (k, v) in enumerate(zip(ks, vs)):
        qb = q[b:b + 1].double().cpu().numpy()
        kb, vb = (x[None].double().cpu().numpy() for x in (k, v))
        out.append(oa.reference_cross_attention(qb, kb, vb, 1 / np.sqrt(q.shape[-1]), False))
    return np.concatenate(out)


def test_block_get_set_data(device):
    # tests/cache/test_block_allocator.py:97-119
    a = BlockAllocator(BlockConfig(block_size=16, num_heads=8, head_dim=64), 10, device=device)
    b = a.allocate(1)[0]
    k, v = rnd((8, 8, 64), 1), rnd((8, 8, 64), 2)
    assert a.set_block_data(b, k, v, start_pos=0, length=8) == b
    k_out, v_out = a.get_block_data(b)
    torch.cuda.synchronize()
    assert torch.equal(k_out[:8], k) and torch.equal(v_out[:8], v)
    assert not k_out[8:].any()


def test_block_copy_on_write_copies_data(device):
    # test_block_allocator.py:121-141, with the data checked
    a = BlockAllocator(BlockConfig(block_size=16, num_heads=8, head_dim=64), 10, device=device)
    b = a.allocate(1)[0]
    k = torch.ones((16, 8, 64), dtype=torch.float16, device=device)
    a.set_block_data(b, k, 2 * k)
    a.increment_ref(b)
    nb = a.set_block_data(b, 3 * k[:4], 4 * k[:4], start_pos=2)
    assert nb != b and a.get_ref_count(b) == 1
    torch.cuda.synchronize()
    old_k, old_v = a.get_block_data(b)
    new_k, new_v = a.get_block_data(nb)
    assert torch.equal(old_k, k) and torch.equal(old_v, 2 * k)  # shared block untouched
    assert torch.equal(new_k[2:6], 3 * k[:4]) and torch.equal(new_k[:2], k[:2])
    assert torch.equal(new_v[6:], 2 * k[6:])


def test_cache_then_paged_attention(device):
    # tests/cache/test_paged_attention.py:339-364
    c = cache(device)
    sid = c.create_sequence()
    k, v = rnd((32, 8, 64), 3), rnd((32, 8, 64), 4)
    c.update(sid, k, v, layer_idx=0)
    k_pool, v_pool, tables, lens = c.get_kv_paged([sid], layer_idx=0)
    assert tables.dtype == torch.int32 and lens.tolist() == [32]
    q = rnd((1, 1, 8, 64), 5)
    out = paged_attention(q, k_pool, v_pool, tables, lens, block_size=16)
    assert out.shape == (1, 1, 8, 64)
    err = np.abs(out.double().cpu().numpy() - decode_ref(q, [k], [v])).max()
    assert err <= 2e-2, err


def test_batched_cache_attention_and_incremental_decode(device):
    # tests/cache/test_paged_attention.py:366-395, then decode steps appending one
    # token per sequence with update_batch
    c = cache(device, gb=0.5)
    lengths = [20, 35, 50]
    ids, ks, vs = [], [], []
    for i, n in enumerate(lengths):
        sid = c.create_sequence()
        k, v = rnd((n, 8, 64), 10 + i), rnd((n, 8, 64), 20 + i)
        c.update(sid, k, v, layer_idx=0)
        ids.append(sid)
        ks.append(k)
        vs.append(v)
    errors = torch.zeros(3, dtype=torch.int32, device=device)
    for step in range(20):
        nk, nv = rnd((3, 1, 8, 64), 100 + step), rnd((3, 1, 8, 64), 200 + step)
        c.update_batch(ids, nk, nv, layer_idx=0, errors=errors)
        ks = [torch.cat([k, nk[b]]) for b, k in enumerate(ks)]
        vs = [torch.cat([v, nv[b]]) for b, v in enumerate(vs)]
        q = rnd((3, 1, 8, 64), 300 + step)
        k_pool, v_pool, tables, lens = c.get_kv_paged(ids, layer_idx=0)
        out = paged_attention(q, k_pool, v_pool, tables, lens, block_size=16)
        err = np.abs(out.double().cpu().numpy() - decode_ref(q, ks, vs)).max()
        assert err <= 2e-2, (step, err)
    assert errors.tolist() == [0, 0, 0]
    assert lens.tolist() == [n + 20 for n in lengths]
    for sid, k, v in zip(ids, ks, vs):
        gk, gv = c.get_kv(sid, 0)
        assert torch.equal(gk, k) and torch.equal(gv, v)


def test_fork_then_append_keeps_parent(device):
    # Copy-on-write at the table: the fork's tokens go to its own copy of the
    # shared last page; the parent's pages are unchanged.
    c = cache(device, num_layers=2)
    parent = c.create_sequence()
    k, v = rnd((40, 8, 64), 30), rnd((40, 8, 64), 31)
    for layer in range(2):
        c.update(parent, k, v, layer)
    child = c.fork_sequence(parent)
    k2, v2 = rnd((30, 8, 64), 32), rnd((30, 8, 64), 33)
    for layer in range(2):
        c.update(child, k2, v2, layer)
    k3, v3 = rnd((5, 8, 64), 34), rnd((5, 8, 64), 35)
    c.update(parent, k3, v3, 1)
    for layer in range(2):
        ck, cv = c.get_kv(child, layer)
        assert torch.equal(ck, torch.cat([k, k2])) and torch.equal(cv, torch.cat([v, v2]))
        pk, pv = c.get_kv(parent, layer)
        want_k = torch.cat([k, k3]) if layer == 1 else k
        want_v = torch.cat([v, v3]) if layer == 1 else v
        assert torch.equal(pk, want_k) and torch.equal(pv, want_v)
    # the first two pages are still shared, the third was copied
    t_parent = c.get_kv_paged([parent], 0)[2][0].tolist()
    t_child = c.get_kv_paged([child], 0)[2][0].tolist()
    assert t_parent[:2] == t_child[:2] and t_parent[2] != t_child[2]


def test_rollback_update_at_position(device):
    # update(position=...) truncates and rewrites (speculative decoding rollback)
    c = cache(device)
    sid = c.create_sequence()
    k, v = rnd((50, 8, 64), 40), rnd((50, 8, 64), 41)
    c.update(sid, k, v, 0)
    kr, vr = rnd((7, 8, 64), 42), rnd((7, 8, 64), 43)
    c.update(sid, kr, vr, 0, position=30)
    gk, gv = c.get_kv(sid, 0)
    assert c.get_sequence_length(sid) == 37
    assert torch.equal(gk, torch.cat([k[:30], kr])) and torch.equal(gv, torch.cat([v[:30], vr]))


def test_create_sequence_with_initial_kv_and_wrapper(device):
    c = cache(device, num_layers=3)
    k, v = rnd((21, 8, 64), 50), rnd((21, 8, 64), 51)
    sid = c.create_sequence(k, v)
    for layer in range(3):
        gk, gv = c.get_kv(sid, layer)
        assert torch.equal(gk, k) and torch.equal(gv, v)
    m = MultiLayerKVCache.from_model_config(num_layers=2, num_heads=4, head_dim=32,
                                            max_memory_gb=0.01, block_size=8, device=device)
    s = m.create_sequence()
    a, b = rnd((3, 4, 32), 52), rnd((3, 4, 32), 53)
    gk, gv = m.get_or_update(s, 1, a, b)
    gk2, gv2 = m.get_or_update(s, 1, b, a)
    assert torch.equal(gk2, torch.cat([a, b])) and torch.equal(gv2, torch.cat([b, a]))


def test_store_errors_from_host_checks(device):
    c = cache(device)
    sid = c.create_sequence()
    k, v = rnd((10, 8, 64), 60), rnd((10, 8, 64), 61)
    c.update(sid, k, v, 0)
    with pytest.raises(ValueError, match="write_start"):
        c._store_kv(sid, rnd((20, 8, 64), 62), rnd((20, 8, 64), 63), 0)
    # past the table: the tokens that fit are written, then RuntimeError
    with pytest.raises(RuntimeError, match="out of range"):
        c._store_kv(sid, k, v, 0, start_position=12)
    gk, _ = c.get_kv(sid, 0)
    blk, slot = 0, 12
    k_pool = c.get_kv_paged([sid], 0)[0]
    table = c.get_kv_paged([sid], 0)[2][0].tolist()
    assert torch.equal(k_pool[table[blk], slot:16], k[:4])


def test_update_batch_ragged_matches_updates(device):
    c1, c2 = cache(device), cache(device)
    ids1 = [c1.create_sequence() for _ in range(4)]
    ids2 = [c2.create_sequence() for _ in range(4)]
    counts = [5, 0, 17, 9]
    k, v = rnd((4, 17, 8, 64), 70), rnd((4, 17, 8, 64), 71)
    c1.update_batch(ids1, k, v, 0, num_tokens=counts)
    for b, n in enumerate(counts):
        c2.update(ids2[b], k[b, :n], v[b, :n], 0)
    for s1, s2, n in zip(ids1, ids2, counts):
        a, b_ = c1.get_kv(s1, 0), c2.get_kv(s2, 0)
        assert a[0].shape[0] == n and torch.equal(a[0], b_[0]) and torch.equal(a[1], b_[1])

"""RoPE on the serving path: K rotated as it is appended to the paged cache
(store_kv / KVCache with rope=...) and queries rotated at each sequence's own
position (rope_at), so paged attention over the cache needs no separate K pass.

Bit-for-bit: the append kernel's K pages against rope(k, offset=start) stored
by the plain append, and rope_at against per-sequence rope calls (all three
kernels round the same float32 rotation once). Against the oracle: a decode
loop over a rotated cache against float64 attention over oracle-rotated Q and
K (fp16: max-abs 2e-2). The reference has no cache-side rotation
(kernels/fused_rope_attention.py:766-800 rotates K at kv_offset + j inside
attention); its positions are the ones used here.
"""

import numpy as np
import pytest
import torch

from mlx_primitives.cache import KVCache, KVCacheConfig, paged_attention
from mlx_primitives.cache.kv_store import store_kv
from mlx_primitives.kernels import precompute_rope_cache, rope, rope_at
from oracle import attention as oa
from oracle import rope as orope

pytestmark = pytest.mark.gpu


def rnd(shape, seed, dtype, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype).to(device)


def pools(num_blocks, bs, H, D, dtype, device):
    z = torch.zeros((num_blocks, bs, H, D), dtype=dtype, device=device)
    return z, z.clone()


@pytest.mark.parametrize("dtype,cache_dtype", [(torch.bfloat16, torch.float32),
                                               (torch.float16, torch.float16),
                                               (torch.float32, torch.float32)])
def test_store_kv_rope_matches_rope_then_store(device, dtype, cache_dtype):
    B, T, H, D, bs = 3, 37, 4, 64, 16
    n_pos = 160
    cos, sin = precompute_rope_cache(n_pos, D, dtype=cache_dtype, device=device)
    k, v = rnd((B, T, H, D), 1, dtype), rnd((B, T, H, D), 2, dtype)
    starts = [0, 5, 100]
    counts = [37, 20, 31]
    max_blocks = (n_pos + bs - 1) // bs
    perm = torch.randperm(B * max_blocks, generator=torch.Generator().manual_seed(3))
    tables = perm.view(B, max_blocks).to(torch.int32).to(device)
    kp1, vp1 = pools(B * max_blocks, bs, H, D, dtype, device)
    kp2, vp2 = pools(B * max_blocks, bs, H, D, dtype, device)
    store_kv(kp1, vp1, tables, k, v, torch.tensor(starts, dtype=torch.int32),
             torch.tensor(counts, dtype=torch.int32), rope=(cos, sin))
    k_rot = torch.stack([rope(k[b:b + 1], cos, sin, offset=starts[b])[0] for b in range(B)])
    store_kv(kp2, vp2, tables, k_rot, v, torch.tensor(starts, dtype=torch.int32),
             torch.tensor(counts, dtype=torch.int32))
    torch.cuda.synchronize()
    assert torch.equal(kp1, kp2)
    assert torch.equal(vp1, vp2)
    # the rows really were rotated (sequence 1 starts at position 5)
    assert not torch.equal(k_rot[1, :1], k[1, :1])


def test_store_kv_rope_errors(device):
    B, T, H, D, bs = 2, 8, 2, 32, 8
    cos, sin = precompute_rope_cache(16, D, device=device)
    k = rnd((B, T, H, D), 4, torch.float16)
    kp, vp = pools(8, bs, H, D, torch.float16, device)
    tables = torch.arange(8, dtype=torch.int32, device=device).view(B, 4)
    with pytest.raises(ValueError, match="RoPE position"):
        store_kv(kp, vp, tables, k, k, torch.tensor([0, 12], dtype=torch.int32), rope=(cos, sin))
    err = store_kv(kp, vp, tables, k, k, torch.tensor([0, 12], dtype=torch.int32),
                   rope=(cos, sin), check=False)
    assert err.tolist() == [0, 0, 0, 1]
    # the first sequence's tokens and the second's that fit were written
    torch.cuda.synchronize()
    assert kp[0].abs().sum() > 0
    errors = torch.full((4,), 7, dtype=torch.int32, device=device)
    store_kv(kp, vp, tables, k, k, 0, rope=(cos, sin), check=False, errors=errors)
    assert errors.tolist() == [0, 0, 0, 0]
    with pytest.raises(ValueError, match="4 entries"):
        store_kv(kp, vp, tables, k, k, 0, rope=(cos, sin), errors=torch.zeros(
            3, dtype=torch.int32, device=device))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_at_matches_per_sequence_rope(device, dtype):
    B, S, H, D = 4, 3, 8, 128
    cos, sin = precompute_rope_cache(64, D, device=device)
    x = rnd((B, S, H, D), 5, dtype)
    pos = [0, 7, 33, 61]
    got = rope_at(x, cos, sin, pos)
    want = torch.cat([rope(x[b:b + 1], cos, sin, offset=pos[b]) for b in range(B)])
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    # float64 oracle
    c64, s64 = orope.precompute_rope_cache(64, D, dtype=np.float64)
    xo = x.double().cpu().numpy()
    ref = np.concatenate([orope.rope(xo[b:b + 1], c64, s64, pos[b]) for b in range(B)])
    # float32: the tables' own rounding (angle t * inv_freq in float32) moves
    # the rotation by ~1e-7 t rad against the float64 tables
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert np.abs(got.double().cpu().numpy() - ref).max() <= tol
    with pytest.raises(ValueError, match="outside"):
        rope_at(x, cos, sin, [0, 0, 0, 62])
    errors = torch.zeros(1, dtype=torch.int32, device=device)
    rope_at(x, cos, sin, [0, 0, -1, 0], check=False, errors=errors)
    assert errors.item() == 1


def test_decode_over_rotated_cache(device):
    # A serving loop: prompts appended with K rotated, then decode steps that
    # rotate each new query at its sequence's position and append its K/V.
    H, D, bs, n_pos = 8, 64, 16, 256
    cfg = KVCacheConfig(num_heads=H, head_dim=D, num_layers=1, max_memory_gb=0.1,
                        block_size=bs)
    cache = KVCache(cfg, device=device)
    cos, sin = precompute_rope_cache(n_pos, D, device=device)
    c64, s64 = orope.precompute_rope_cache(n_pos, D, dtype=np.float64)
    lengths = [19, 40, 7]
    ids, ks, vs = [], [], []
    for i, n in enumerate(lengths):
        sid = cache.create_sequence()
        k, v = rnd((n, H, D), 10 + i, torch.float16), rnd((n, H, D), 20 + i, torch.float16)
        cache.update(sid, k, v, 0, rope=(cos, sin))
        ids.append(sid)
        ks.append(k)
        vs.append(v)
    for step in range(6):
        nk = rnd((3, 1, H, D), 100 + step, torch.float16)
        nv = rnd((3, 1, H, D), 200 + step, torch.float16)
        cache.update_batch(ids, nk, nv, 0, rope=(cos, sin))
        ks = [torch.cat([k, nk[b]]) for b, k in enumerate(ks)]
        vs = [torch.cat([v, nv[b]]) for b, v in enumerate(vs)]
        q = rnd((3, 1, H, D), 300 + step, torch.float16)
        k_pool, v_pool, tables, lens = cache.get_kv_paged(ids, 0)
        q_rot = rope_at(q, cos, sin, lens - 1)
        out = paged_attention(q_rot, k_pool, v_pool, tables, lens, block_size=bs)
        for b in range(3):
            n = ks[b].shape[0]
            qo = orope.rope(q[b:b + 1].double().cpu().numpy(), c64, s64, n - 1)
            ko = orope.rope(ks[b][None].double().cpu().numpy(), c64, s64, 0)
            ref = oa.reference_cross_attention(qo, ko, vs[b][None].double().cpu().numpy(),
                                               1 / np.sqrt(D), False)
            err = np.abs(out[b:b + 1].double().cpu().numpy() - ref).max()
            assert err <= 2e-2, (step, b, err)
    # the cache holds rotated K: reading it back equals rope over positions 0..n-1
    gk, gv = cache.get_kv(ids[1], 0)
    assert torch.equal(gk, rope(ks[1][None], cos, sin, 0)[0])
    assert torch.equal(gv, vs[1])


def test_update_rope_position_check_before_mutation(device):
    cfg = KVCacheConfig(num_heads=2, head_dim=32, num_layers=1, max_memory_gb=0.01,
                        block_size=8)
    cache = KVCache(cfg, device=device)
    cos, sin = precompute_rope_cache(10, 32, device=device)
    sid = cache.create_sequence()
    k = rnd((8, 2, 32), 30, torch.float16)
    cache.update(sid, k, k, 0, rope=(cos, sin))
    with pytest.raises(ValueError, match="RoPE position"):
        cache.update(sid, k[:3], k[:3], 0, rope=(cos, sin))
    assert cache.get_sequence_length(sid) == 8
    with pytest.raises(ValueError, match="RoPE position"):
        cache.update_batch([sid], k[None, :3], k[None, :3], 0, rope=(cos, sin))
    assert cache.get_sequence_length(sid) == 8

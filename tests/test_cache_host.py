"""KV-cache bookkeeping on the host (no GPU): BlockConfig, BlockAllocator,
PageTable, KVCacheConfig and the KVCache sequence management, following the
reference's cache tests (tests/cache/test_block_allocator.py:15-336) and its
table formats (cache/page_table.py:295-345)."""

import pytest
import torch

from mlx_primitives.cache import (
    BlockAllocator,
    BlockConfig,
    KVCache,
    KVCacheConfig,
    PageTable,
    calculate_num_blocks,
    get_optimal_block_size,
)

CPU = torch.device("cpu")


def alloc(num_blocks=100, **kw):
    return BlockAllocator(BlockConfig(block_size=16, num_heads=8, head_dim=64), num_blocks,
                          device=CPU, **kw)


# ---- BlockConfig (test_block_allocator.py:15-42) --------------------------------

def test_block_config_defaults_and_sizes():
    c = BlockConfig()
    assert (c.block_size, c.num_heads, c.head_dim) == (16, 32, 128)
    assert BlockConfig(block_size=16, num_heads=8, head_dim=64).block_bytes == 32768
    assert BlockConfig(16, 8, 64, torch.float32).block_bytes == 65536
    assert BlockConfig(16, 8, 64).kv_shape == (16, 8, 64)
    assert BlockConfig(16, 8, 64).tokens_per_block == 16


# ---- BlockAllocator (test_block_allocator.py:44-176) ----------------------------

def test_allocate_free_reallocate():
    a = alloc(100)
    blocks = a.allocate(5)
    assert len(blocks) == 5 and len(set(blocks)) == 5
    assert (a.num_allocated_blocks, a.num_free_blocks) == (5, 95)
    more = a.allocate(5)
    a.free(blocks)
    assert (a.num_allocated_blocks, a.num_free_blocks) == (5, 95)
    again = a.allocate(3)
    assert set(again) <= set(blocks)  # freed blocks come back first
    assert a.num_allocated_blocks == 8
    assert not set(again) & set(more)


def test_allocate_all_and_beyond():
    a = alloc(10)
    assert sorted(a.allocate(10)) == list(range(10))
    assert a.num_free_blocks == 0
    with pytest.raises(RuntimeError, match="Cannot allocate"):
        alloc(5).allocate(10)


def test_free_validation_and_unallocated_ignored():
    a = alloc(10)
    with pytest.raises(ValueError, match="out of bounds"):
        a.free([10])
    with pytest.raises(ValueError, match="out of bounds"):
        a.free([-1])
    a.free([3])  # not allocated: ignored
    assert a.num_free_blocks == 10


def test_reference_counts_and_copy_on_write_bookkeeping():
    a = alloc(10, enable_cow=True)
    b = a.allocate(1)[0]
    a.increment_ref(b)
    assert a.get_ref_count(b) == 2
    a.free([b])  # one sharer left: still allocated
    assert a.get_ref_count(b) == 1 and a.num_allocated_blocks == 1
    assert a.copy_on_write(b) == b  # single owner: modify in place
    a.increment_ref(b)
    nb = a.copy_on_write(b)
    assert nb != b and a.get_ref_count(b) == 1 and a.get_ref_count(nb) == 1
    no_cow = alloc(10, enable_cow=False)
    c = no_cow.allocate(1)[0]
    no_cow.increment_ref(c)
    assert no_cow.copy_on_write(c) == c


def test_pools_clear_and_stats():
    a = alloc(100)
    k, v = a.get_pools()
    assert k.shape == v.shape == (100, 16, 8, 64) and k.dtype == torch.float16
    a.allocate(25)
    st = a.get_stats()
    assert (st["num_blocks"], st["num_allocated"], st["num_free"], st["utilization"]) == (
        100, 25, 75, 0.25)
    assert a.memory_usage_bytes == 25 * 32768 and a.total_memory_bytes == 100 * 32768
    a.clear()
    assert (a.num_allocated_blocks, a.num_free_blocks) == (0, 100)


# ---- PageTable (test_block_allocator.py:178-311) --------------------------------

def test_page_table_create_extend_truncate():
    a = alloc(100)
    pt = PageTable(a)
    sid = pt.create_sequence()
    assert sid == 0 and pt.num_sequences == 1
    s2 = pt.create_sequence(initial_tokens=48)
    assert len(pt.get_sequence_metadata(s2).block_table) == 3
    assert pt.get_sequence_metadata(s2).num_tokens == 0
    pt.extend_sequence(sid, 20)
    m = pt.get_sequence_metadata(sid)
    assert (m.num_tokens, len(m.block_table), m.num_tokens_in_last_block) == (20, 2, 4)
    for _ in range(12):
        pt.extend_sequence(sid, 1)
    assert (m.num_tokens, len(m.block_table), m.num_tokens_in_last_block) == (32, 2, 16)
    pt.extend_sequence(s2, 48)  # fits the reserved blocks
    assert len(pt.get_sequence_metadata(s2).block_table) == 3
    before = a.num_allocated_blocks
    pt.truncate_sequence(s2, 20)
    m2 = pt.get_sequence_metadata(s2)
    assert (m2.num_tokens, len(m2.block_table)) == (20, 2)
    assert a.num_allocated_blocks == before - 1
    pt.truncate_sequence(s2, 0)
    assert pt.get_sequence_metadata(s2).block_table == []
    with pytest.raises(KeyError):
        pt.extend_sequence(99, 1)


def test_page_table_fork_delete_and_positions():
    a = alloc(100, enable_cow=True)
    pt = PageTable(a)
    sid = pt.create_sequence(initial_tokens=32)
    pt.extend_sequence(sid, 32)
    fid = pt.fork_sequence(sid)
    assert fid != sid and pt.num_sequences == 2
    assert pt.get_block_table(sid) == pt.get_block_table(fid)
    assert all(a.get_ref_count(b) == 2 for b in pt.get_block_table(sid))
    # the fork writes its last block: it gets a private copy, the parent keeps its own
    pt.make_writable(fid, 1, 1)
    assert pt.get_block_table(fid)[0] == pt.get_block_table(sid)[0]
    assert pt.get_block_table(fid)[1] != pt.get_block_table(sid)[1]
    blk, slot = pt.get_token_position(sid, 20)
    assert (blk, slot) == (pt.get_block_table(sid)[1], 4)
    allocated = a.num_allocated_blocks
    pt.delete_sequence(sid)
    assert pt.num_sequences == 1 and a.num_allocated_blocks == allocated - 1
    pt.delete_sequence(12345)  # unknown: ignored


def test_block_table_tensor_and_context_lengths():
    a = alloc(100)
    pt = PageTable(a)
    s1 = pt.create_sequence()
    pt.extend_sequence(s1, 16)
    s2 = pt.create_sequence()
    pt.extend_sequence(s2, 48)
    s3 = pt.create_sequence()
    pt.extend_sequence(s3, 35)
    t = pt.get_block_table_tensor([s1, s2, s3])
    assert t.dtype == torch.int32 and tuple(t.shape) == (3, 3)
    assert t[0, 1:].tolist() == [-1, -1] and t[2, 2] >= 0
    assert t[1].tolist() == pt.get_block_table(s2)
    cut = pt.get_block_table_tensor([s2], max_blocks=2)
    assert cut.tolist() == [pt.get_block_table(s2)[:2]]
    wide = pt.get_block_table_tensor([s1], max_blocks=4)
    assert wide[0, 1:].tolist() == [-1, -1, -1]
    lens = pt.get_context_lengths([s1, s2, s3])
    assert lens.dtype == torch.int32 and lens.tolist() == [16, 48, 35]
    assert pt.get_block_table_tensor([]).numel() == 0
    st = pt.get_stats()
    assert (st["num_sequences"], st["total_tokens"], st["total_blocks"]) == (3, 99, 7)


# ---- utilities (test_block_allocator.py:313-336) ---------------------------------

def test_optimal_block_size_and_num_blocks():
    bs = get_optimal_block_size(head_dim=128, num_heads=32, dtype=torch.float16)
    assert bs in (8, 16, 32, 64) and bs & (bs - 1) == 0
    # 4 MB L2 x 0.5 / 4 blocks = 512 KB per block; 16 KB per token -> 32
    assert bs == 32
    assert get_optimal_block_size(64, 8, torch.float16, l2_cache_mb=1024.0) == 64
    assert get_optimal_block_size(128, 128, torch.float32, l2_cache_mb=0.5) == 8
    cfg = BlockConfig(block_size=16, num_heads=8, head_dim=64)
    assert calculate_num_blocks(0.1, cfg) == int(0.1 * 1e9 * 0.9 / cfg.block_bytes)


# ---- KVCache bookkeeping ---------------------------------------------------------------

def small_cache(**kw):
    cfg = KVCacheConfig(num_heads=8, head_dim=64, num_layers=2, max_memory_gb=0.02,
                        block_size=16, **kw)
    return KVCache(cfg, device=CPU)


def test_kv_cache_config_capacity():
    cfg = KVCacheConfig(num_heads=8, head_dim=64, num_layers=2, max_memory_gb=0.02,
                        block_size=16)
    blocks, tokens = cfg.calculate_capacity()
    assert blocks == int(0.01 * 1e9 * 0.9 / 32768) and tokens == blocks * 16
    assert KVCacheConfig(num_heads=32, head_dim=128, num_layers=1).block_size == 32


def test_kv_cache_sequences_fork_delete_stats():
    c = small_cache()
    a, b = c.create_sequence(), c.create_sequence()
    assert c.get_all_sequence_ids() == [a, b] and c.get_sequence_length(a) == 0
    f = c.fork_sequence(a)
    assert f not in (a, b)
    st = c.memory_stats
    assert st.num_sequences == 3 and st.num_blocks_allocated == 0 and st.utilization == 0.0
    c.delete_sequence(b)
    assert c.get_all_sequence_ids() == [a, f]
    with pytest.raises(KeyError):
        c.delete_sequence(b)
    with pytest.raises(KeyError):
        c.get_kv_paged([b], 0)
    k, v = c.get_kv(a, 1)
    assert k.shape == (0, 8, 64)
    pools_k, pools_v, tables, lens = c.get_kv_paged([a, f], 0)
    assert pools_k.shape[1:] == (16, 8, 64) and lens.tolist() == [0, 0]
    c.clear()
    assert c.get_all_sequence_ids() == [] and c.memory_stats.num_blocks_allocated == 0


def test_kv_cache_lru_eviction():
    c = small_cache()
    ids = [c.create_sequence() for _ in range(3)]
    # reserve blocks through the page tables (bookkeeping only)
    for layer in range(2):
        for s in ids:
            c._page_tables[layer].extend_sequence(c._sequence_ids[s][layer], 16 * 50)
    c._notify("on_access", ids[0])  # ids[1] is now the oldest
    total = c.memory_stats.total_bytes
    used = c.memory_stats.used_bytes
    n = c.evict_if_needed(total - used + 1, protected_sequences=[ids[1]])
    assert n == 1 and ids[1] in c.get_all_sequence_ids() and ids[2] not in c.get_all_sequence_ids()
    assert c.evict_if_needed(0) == 0


def test_kv_cache_update_batch_rolls_back_when_the_pool_runs_out():
    # Three 100-block appends into 274 free blocks: the third cannot allocate,
    # and the two sequences already extended go back to their lengths, so no
    # sequence counts tokens that were never written.
    c = small_cache()
    ids = [c.create_sequence() for _ in range(3)]
    free = c._allocators[0].num_free_blocks
    T = 16 * 100
    assert 2 * 100 <= free < 3 * 100
    k = torch.zeros((3, T, 8, 64), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="Cannot allocate"):
        c.update_batch(ids, k, k, 0)
    assert [c.get_sequence_length(s) for s in ids] == [0, 0, 0]
    assert c._allocators[0].num_free_blocks == free
    with pytest.raises(ValueError, match="distinct"):
        c.update_batch([ids[0], ids[0]], k[:2], k[:2], 0)


def test_kv_cache_update_rolls_back_a_failed_copy_on_write():
    # A shared, partly filled last block needs a private copy before the next
    # token is written; with the pool empty the copy fails and the sequence
    # keeps its length and its table.
    c = small_cache()
    a = c.create_sequence()
    pt, alloc = c._page_tables[0], c._allocators[0]
    lsid = c._sequence_ids[a][0]
    pt.extend_sequence(lsid, 150)
    c.fork_sequence(a)
    table = pt.get_block_table(lsid)
    alloc.allocate(alloc.num_free_blocks)
    one = torch.zeros((1, 8, 64), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="Cannot allocate"):
        c.update(a, one, one, 0)
    assert c.get_sequence_length(a) == 150 and pt.get_block_table(lsid) == table

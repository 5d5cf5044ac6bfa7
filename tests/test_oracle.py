"""Pins of the CPU oracle (oracle/attention.py, oracle/attention_grad.py,
oracle/paged.py, oracle/kv_cache.py, oracle/rope.py).

Each oracle function is checked against something that does not restate it:
  * known-answer cases from the reference's own tests (cited file:line);
  * an independent brute-force evaluation (per-row Python loops, math.exp)
    on tiny inputs;
  * torch.nn.functional.scaled_dot_product_attention in float64 (the routine
    the reference's parity suite compares with,
    tests/parity/pytorch/test_attention_parity.py:87-105);
  * invariants: block/chunk-size independence, merge associativity, full
    window == causal, large/small input scales, KV append write-then-gather
    round trips;
  * for the gradients: torch autograd in float64 (masks built independently,
    K/V heads expanded with repeat_interleave), torch's SDPA backward and
    central finite differences of the pinned forward.
The last group plants mistakes in the oracle and checks a pin catches each.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oa
from oracle import attention_grad as oag
from oracle import kv_cache as ok
from oracle import paged as op
from oracle import rope as orope


def rnd(shape, seed, dtype=np.float64):
    return np.random.default_rng(seed).standard_normal(shape).astype(dtype)


def brute_attention(q, k, v, scale, allowed, eps=0.0):
    """q (B,Sq,H,D), k/v (B,Sk,H,D); allowed(i, j) -> bool. Pure loops."""
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    out = np.zeros((B, Sq, H, v.shape[3]))
    for b in range(B):
        for h in range(H):
            for i in range(Sq):
                js = [j for j in range(Sk) if allowed(i, j)]
                s = [sum(float(q[b, i, h, d]) * float(k[b, j, h, d]) for d in range(D)) * scale
                     for j in js]
                m = max(s)
                w = [math.exp(x - m) for x in s]
                tot = sum(w)
                for wi, j in zip(w, js):
                    out[b, i, h] += wi * v[b, j, h].astype(np.float64)
                out[b, i, h] /= (tot + eps)
    return out


def sdpa(q, k, v, scale, mask=None):
    """torch SDPA in float64 on BSHD numpy arrays; mask (Sq, Sk) bool."""
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).double().transpose(1, 2)
    m = None if mask is None else torch.from_numpy(mask)
    out = F.scaled_dot_product_attention(t(q), t(k), t(v), attn_mask=m, scale=scale)
    return out.transpose(1, 2).numpy()


def causal_mask(sq, sk):
    return np.arange(sk)[None, :] <= np.arange(sq)[:, None]


def window_mask(s, w, causal):
    i, j = np.arange(s)[:, None], np.arange(s)[None, :]
    m = np.abs(i - j) <= w
    return m & (j <= i) if causal else m


# ---- known answers from the reference's tests ---------------------------------

@pytest.mark.parametrize("block", [1, 2, 4, 32])
def test_attention_identity_kat(block):
    # tests/reference.py:453-468: q = k = 1, v = [1,2,3,4] -> [1, 1.5, 2, 2.5].
    q = np.ones((1, 4, 1, 1))
    v = np.array([1.0, 2.0, 3.0, 4.0]).reshape(1, 4, 1, 1)
    out = oa.tiled_flash_attention(q, q.copy(), v, 1.0, True, block, block)
    np.testing.assert_allclose(out.ravel(), [1.0, 1.5, 2.0, 2.5], rtol=1e-5)
    dense = oa.dense_attention_bhsd(q.transpose(0, 2, 1, 3), q.transpose(0, 2, 1, 3),
                                    v.transpose(0, 2, 1, 3), 1.0, True)
    np.testing.assert_allclose(dense.ravel(), [1.0, 1.5, 2.0, 2.5], rtol=1e-12)


def test_single_token_returns_v():
    # tests/attention/test_flash.py:217-230
    q, k, v = (rnd((2, 1, 4, 64), s) for s in (1, 2, 3))
    out = oa.flash_attention(q, k, v, causal=True)
    np.testing.assert_allclose(out, v, rtol=1e-5, atol=1e-6)


def test_first_position_sees_only_self():
    # tests/attention/test_metal_python_parity.py:159-184
    q = np.zeros((1, 16, 2, 32)); k = np.zeros((1, 16, 2, 32)); v = np.ones((1, 16, 2, 32))
    q[:, 0] = 1.0; k[:, 0] = 1.0
    out = oa.flash_attention(q, k, v, causal=True)
    np.testing.assert_allclose(out[:, 0], 1.0, rtol=1e-4, atol=1e-4)


def test_uniform_attention_mean():
    # tests/attention/test_metal_python_parity.py:207-232
    seq = 64
    q = np.ones((1, seq, 2, 32)); k = np.ones((1, seq, 2, 32))
    v = np.broadcast_to(np.arange(seq, dtype=np.float64).reshape(1, seq, 1, 1), (1, seq, 2, 32)).copy()
    out = oa.flash_attention(q, k, v, causal=False)
    np.testing.assert_allclose(out.mean(), (seq - 1) / 2.0, rtol=1e-2)


def test_window_restriction_kat():
    # tests/attention/test_sliding_window.py:216-233
    q = np.zeros((1, 16, 1, 8)); k = np.zeros((1, 16, 1, 8)); v = np.zeros((1, 16, 1, 8))
    q[0, 0, 0, 0] = 1.0; k[0, 15, 0, 0] = 1.0; v[0, 15, 0, 0] = 100.0
    out = oa.sliding_window_attention(q, k, v, window_size=4, causal=False)
    assert abs(out[0, 0, 0, 0]) < 1.0


def test_full_window_equals_causal():
    # tests/attention/test_sliding_window.py:192-211
    q, k, v = (rnd((2, 16, 2, 32), s) for s in (4, 5, 6))
    sw = oa.sliding_window_attention(q, k, v, window_size=16, causal=True)
    ref = sdpa(q, k, v, 1 / math.sqrt(32), causal_mask(16, 16))
    np.testing.assert_allclose(sw, ref, rtol=1e-5, atol=1e-6)


def test_merge_two_chunks_kat():
    # tests/attention/test_flash.py:395-441: two chunks merged == full attention
    q = rnd((2, 8, 4, 32), 7); k = rnd((2, 32, 4, 32), 8); v = rnd((2, 32, 4, 32), 9)
    s = 1 / math.sqrt(32)
    o1, m1, l1 = oa.compute_chunk_attention(q, k[:, :16], v[:, :16], s)
    o2, m2, l2 = oa.compute_chunk_attention(q, k[:, 16:], v[:, 16:], s, kv_offset=16)
    o, _, l = oa.online_softmax_merge(o1, m1, l1, o2, m2, l2)
    np.testing.assert_allclose(o / l[..., None], sdpa(q, k, v, s), rtol=1e-10, atol=1e-12)


def test_merge_large_score_difference_kat():
    # tests/attention/test_flash.py:528-566
    q = rnd((1, 4, 2, 16), 10)
    k = np.concatenate([rnd((1, 8, 2, 16), 11) * 5, rnd((1, 8, 2, 16), 12) * 0.1], axis=1)
    v = rnd((1, 16, 2, 16), 13)
    s = 0.25
    o1, m1, l1 = oa.compute_chunk_attention(q, k[:, :8], v[:, :8], s)
    o2, m2, l2 = oa.compute_chunk_attention(q, k[:, 8:], v[:, 8:], s, kv_offset=8)
    o, _, l = oa.online_softmax_merge(o1, m1, l1, o2, m2, l2)
    np.testing.assert_allclose(o / l[..., None], sdpa(q, k, v, s), rtol=1e-10, atol=1e-12)


# ---- brute force on tiny inputs -------------------------------------------------

@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("block", [1, 2, 3, 32])
def test_tiled_flash_vs_brute(causal, block):
    q, k, v = (rnd((2, 7, 2, 3), s) for s in (20, 21, 22))
    s = 0.7
    out = oa.tiled_flash_attention(q, k, v, s, causal, block, block)
    ref = brute_attention(q, k, v, s, (lambda i, j: j <= i) if causal else (lambda i, j: True),
                          eps=1e-6)
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("w", [0, 1, 3, 9])
def test_sliding_window_vs_brute(causal, w):
    q, k, v = (rnd((1, 9, 2, 3), s) for s in (23, 24, 25))
    s = 0.9
    out = oa.tiled_sliding_window_attention(q, k, v, w, s, causal, block_q=4)
    allowed = (lambda i, j: abs(i - j) <= w and j <= i) if causal else (lambda i, j: abs(i - j) <= w)
    ref = brute_attention(q, k, v, s, allowed, eps=1e-6)
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_chunked_cross_vs_brute(causal):
    q = rnd((1, 5, 2, 3), 26); k = rnd((1, 11, 2, 3), 27); v = rnd((1, 11, 2, 3), 28)
    s = 0.6
    out = oa.chunked_cross_attention(q, k, v, chunk_size=4, scale=s, causal=causal)
    ref = brute_attention(q, k, v, s, (lambda i, j: j <= i) if causal else (lambda i, j: True),
                          eps=1e-6)
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq,skv", [(5, 11), (11, 5), (7, 7), (1, 9)])
def test_reference_cross_dense_branch_vs_brute(causal, sq, skv):
    # Skv <= chunk_size routes to the dense branch (chunked.py:113-114 -> 172-203):
    # exact softmax (no epsilon, so 1e-12 here rejects an O(1e-6) normaliser) and
    # the top-left rule j <= i on absolute positions.
    q = rnd((2, sq, 2, 3), 60); k = rnd((2, skv, 2, 3), 61); v = rnd((2, skv, 2, 3), 62)
    out = oa.chunked_cross_attention(q, k, v, chunk_size=16, scale=0.7, causal=causal)
    ref = brute_attention(q, k, v, 0.7, (lambda i, j: j <= i) if causal else (lambda i, j: True))
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq,skv", [(33, 64), (64, 20)])
def test_reference_cross_dense_branch_vs_sdpa(causal, sq, skv):
    q = rnd((1, sq, 2, 8), 63); k = rnd((1, skv, 2, 8), 64); v = rnd((1, skv, 2, 8), 65)
    out = oa.chunked_cross_attention(q, k, v, chunk_size=64, scale=0.4, causal=causal)
    ref = sdpa(q, k, v, 0.4, causal_mask(sq, skv) if causal else None)
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)


def test_sdpa_causal_rule_kats():
    # utils/masking.py:44-50: one new token over 100 cached keys sees all 100.
    assert oa.sdpa_causal_keep(1, 100).all()
    # Sq <= Sk: the reference's create_causal_mask (triu, k = Sk - Sq + 1) keeps
    # exactly the zero entries of the additive mask.
    for sq, sk in [(4, 4), (3, 8), (1, 5)]:
        np.testing.assert_array_equal(oa.sdpa_causal_keep(sq, sk),
                                      oa.causal_additive_mask(sq, sk) == 0)
    # Sq > Sk: the top-left rule of the tiled path; every row sees key 0.
    np.testing.assert_array_equal(oa.sdpa_causal_keep(6, 3), causal_mask(6, 3))
    assert oa.sdpa_causal_keep(6, 3)[:, 0].all()


@pytest.mark.parametrize("sq,sk", [(5, 12), (12, 5), (9, 9), (1, 7)])
@pytest.mark.parametrize("layout", ["BSHD", "BHSD"])
def test_flash_default_route_vs_brute_and_sdpa(sq, sk, layout):
    q = rnd((2, sq, 3, 8), 66); k = rnd((2, sk, 3, 8), 67); v = rnd((2, sk, 3, 8), 68)
    off = max(0, sk - sq)
    brute = brute_attention(q, k, v, 0.3, lambda i, j: j <= i + off)
    # torch's own causal variants: lower-right aligned for Sk >= Sq, is_causal
    # (upper-left) for Sq > Sk.
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).double().transpose(1, 2)
    if sk >= sq:
        from torch.nn.attention.bias import causal_lower_right
        lib = F.scaled_dot_product_attention(t(q), t(k), t(v), attn_mask=causal_lower_right(sq, sk),
                                             scale=0.3)
    else:
        lib = F.scaled_dot_product_attention(t(q), t(k), t(v), is_causal=True, scale=0.3)
    lib = lib.transpose(1, 2).numpy()
    if layout == "BHSD":
        tr = lambda x: np.ascontiguousarray(x.transpose(0, 2, 1, 3))
        out = oa.flash_attention_default_route(tr(q), tr(k), tr(v), 0.3, True,
                                               layout="BHSD").transpose(0, 2, 1, 3)
    else:
        out = oa.flash_attention_default_route(q, k, v, 0.3, True)
    np.testing.assert_allclose(out, brute, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(out, lib, rtol=1e-12, atol=1e-12)
    if sq == sk:  # the default and CPU routes agree on square causal attention
        np.testing.assert_allclose(oa.flash_attention(q, k, v, 0.3, True, 4, 4), out,
                                   rtol=2e-6, atol=2e-6)


def test_attention_rows_vs_brute():
    q, k, v = (rnd((1, 12, 1, 4), s) for s in (29, 30, 31))
    rows = np.array([0, 5, 11])
    out = oa.attention_rows(q[0, rows, 0], k[0, :, 0], v[0, :, 0], rows, 0.5, True, window_left=4)
    ref = brute_attention(q, k, v, 0.5, lambda i, j: j <= i and i - j <= 4, eps=1e-6)
    np.testing.assert_allclose(out, ref[0, rows, 0], rtol=1e-12, atol=1e-12)


def _brute_paged(q, k_pool, v_pool, tables, lens, scale, bs, slopes=None):
    """Rebuild each sequence's contiguous K/V from its pages, then loop."""
    B, _, H, D = q.shape
    out = np.zeros((B, 1, H, D))
    for b in range(B):
        toks = []
        for t in range(int(lens[b])):
            blk = int(tables[b, t // bs])
            if blk >= 0:
                toks.append((t, blk, t % bs))
        for h in range(H):
            sc = []
            for t, blk, slot in toks:
                x = sum(float(q[b, 0, h, d]) * float(k_pool[blk, slot, h, d]) for d in range(D)) * scale
                if slopes is not None:
                    x += float(slopes[h]) * (t - int(lens[b]))
                sc.append(x)
            m = max(sc)
            w = [math.exp(x - m) for x in sc]
            for wi, (t, blk, slot) in zip(w, toks):
                out[b, 0, h] += wi * v_pool[blk, slot, h]
            out[b, 0, h] /= sum(w)
    return out


@pytest.mark.parametrize("alibi", [False, True])
def test_paged_decode_kat_tables(alibi):
    # tests/cache/test_paged_attention.py:164-197 (tables and lengths)
    rng = np.random.default_rng(32)
    H, D, bs = 2, 4, 16
    q = rng.standard_normal((4, 1, H, D)); kp = rng.standard_normal((20, bs, H, D))
    vp = rng.standard_normal((20, bs, H, D))
    lens = np.array([16, 32, 48, 25], np.int32)
    tables = np.array([[0, -1, -1], [1, 2, -1], [3, 4, 5], [6, 7, -1]], np.int32)
    slopes = op.get_alibi_slopes(H) if alibi else None
    out = op.paged_attention(q, kp, vp, tables, lens, scale=0.5, block_size=bs, alibi_slopes=slopes)
    ref = _brute_paged(q, kp, vp, tables, lens, 0.5, bs, slopes)
    np.testing.assert_allclose(out, ref, rtol=1e-6, atol=1e-7)


def test_paged_decode_single_token_and_invalid_page():
    # ctx = [1] (tests/cache/test_paged_attention.py:232-259) and a -1 page
    # inside the context that must be masked.
    rng = np.random.default_rng(33)
    q = rng.standard_normal((2, 1, 2, 4)); kp = rng.standard_normal((5, 4, 2, 4))
    vp = rng.standard_normal((5, 4, 2, 4))
    lens = np.array([1, 10], np.int32)
    tables = np.array([[3, -1, -1], [0, -1, 2]], np.int32)
    out = op.paged_attention(q, kp, vp, tables, lens, scale=1.0, block_size=4)
    np.testing.assert_allclose(out[0, 0], vp[3, 0], rtol=1e-12)
    ref = _brute_paged(q, kp, vp, tables, lens, 1.0, 4)
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)


def test_paged_decode_empty_context_is_nan():
    q = np.ones((1, 1, 1, 4)); kp = np.ones((2, 4, 1, 4))
    out = op.paged_attention(q, kp, kp, np.array([[0]], np.int32), np.array([0], np.int32),
                             block_size=4)
    assert np.isnan(out).all()


def test_paged_prefill_vs_brute():
    rng = np.random.default_rng(34)
    q = rng.standard_normal((1, 3, 1, 2)); kp = rng.standard_normal((3, 2, 1, 2))
    vp = rng.standard_normal((3, 2, 1, 2))
    tables = np.array([[2, 0]], np.int32); lens = np.array([4], np.int32)
    out = op.paged_attention(q, kp, vp, tables, lens, scale=1.0, block_size=2, causal=True)
    kc = np.concatenate([kp[2], kp[0]])[None]; vc = np.concatenate([vp[2], vp[0]])[None]
    ref = brute_attention(q, kc, vc, 1.0, lambda i, j: j <= i)
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)


def _brute_paged_prefill(q, k_pool, v_pool, tables, lens, scale, bs, causal, slopes=None):
    """Per (b, h, i) loops over the tokens rebuilt page by page."""
    B, Sq, H, D = q.shape
    out = np.full((B, Sq, H, D), np.nan)
    for b in range(B):
        toks = [(t, int(tables[b, t // bs]), t % bs) for t in range(int(lens[b]))
                if int(tables[b, t // bs]) >= 0]
        for h in range(H):
            for i in range(Sq):
                sel = [x for x in toks if not causal or x[0] <= i]
                if not sel:
                    continue
                sc = []
                for t, blk, slot in sel:
                    x = sum(float(q[b, i, h, d]) * float(k_pool[blk, slot, h, d])
                            for d in range(D)) * scale
                    if slopes is not None:
                        x += float(slopes[h]) * (t - i)
                    sc.append(x)
                m = max(sc)
                w = [math.exp(x - m) for x in sc]
                acc = np.zeros(D)
                for wi, (t, blk, slot) in zip(w, sel):
                    acc += wi * v_pool[blk, slot, h]
                out[b, i, h] = acc / sum(w)
    return out


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("alibi", [False, True])
def test_paged_prefill_general_vs_brute(causal, alibi):
    # ragged contexts, a -1 page inside the context, ctx < Sq and ctx > Sq,
    # an empty context (NaN rows)
    rng = np.random.default_rng(35)
    H, D, bs = 2, 3, 4
    q = rng.standard_normal((3, 6, H, D)); kp = rng.standard_normal((7, bs, H, D))
    vp = rng.standard_normal((7, bs, H, D))
    tables = np.array([[4, -1, 1], [6, 0, 2], [3, -1, -1]], np.int32)
    lens = np.array([11, 5, 0], np.int32)
    slopes = op.get_alibi_slopes(H) if alibi else None
    out = op.paged_attention(q, kp, vp, tables, lens, scale=0.7, block_size=bs, causal=causal,
                             alibi_slopes=slopes)
    ref = _brute_paged_prefill(q, kp, vp, tables, lens, 0.7, bs, causal, slopes)
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)
    assert np.isnan(out[2]).all()


def test_paged_prefill_vs_sdpa():
    # gathered contiguous K/V + additive float mask (ALiBi, validity, causal)
    rng = np.random.default_rng(36)
    B, Sq, H, D, bs = 2, 9, 3, 8, 4
    q = rng.standard_normal((B, Sq, H, D)); kp = rng.standard_normal((8, bs, H, D))
    vp = rng.standard_normal((8, bs, H, D))
    tables = np.array([[5, 2, -1, 7], [0, 1, 3, 4]], np.int32)
    lens = np.array([14, 9], np.int32)
    slopes = op.get_alibi_slopes(H)
    out = op.paged_attention(q, kp, vp, tables, lens, scale=0.3, block_size=bs, causal=True,
                             alibi_slopes=slopes)
    for b in range(B):
        idx = [(int(tables[b, t // bs]), t % bs, t) for t in range(tables.shape[1] * bs)]
        kc = np.stack([kp[max(p, 0), s] for p, s, _ in idx])[None]
        vc = np.stack([vp[max(p, 0), s] for p, s, _ in idx])[None]
        T = len(idx)
        mask = np.zeros((H, Sq, T))
        for i in range(Sq):
            for j, (p, s, t) in enumerate(idx):
                if p < 0 or t >= lens[b] or t > i:
                    mask[:, i, j] = -np.inf
                else:
                    mask[:, i, j] = slopes * (t - i)
        ref = F.scaled_dot_product_attention(
            torch.from_numpy(q[b:b + 1]).transpose(1, 2), torch.from_numpy(kc).transpose(1, 2),
            torch.from_numpy(vc).transpose(1, 2), attn_mask=torch.from_numpy(mask)[None],
            scale=0.3).transpose(1, 2).numpy()
        np.testing.assert_allclose(out[b:b + 1], ref, rtol=1e-10, atol=1e-12)


# ---- KV append (oracle/kv_cache.py) ------------------------------------------------

def gather_tokens(pool, table, bs, start, n):
    """Read positions start..start+n-1 back through one block table."""
    return np.stack([pool[table[p // bs], p % bs] for p in range(start, start + n)])


def test_set_get_block_data_kat():
    # tests/cache/test_block_allocator.py:97-119: write 8 tokens at slot 0 of a
    # page, read the page back, the first 8 slots equal the input
    rng = np.random.default_rng(40)
    kp = np.zeros((10, 16, 8, 64), np.float32); vp = np.zeros_like(kp)
    k = rng.standard_normal((8, 8, 64)).astype(np.float32); v = -k
    ok.set_block_data(kp, vp, 3, k, v, start_pos=0, length=8)
    np.testing.assert_array_equal(kp[3, :8], k)
    np.testing.assert_array_equal(vp[3, :8], v)
    assert not kp[3, 8:].any() and not np.delete(kp, 3, axis=0).any()


@pytest.mark.parametrize("start,n", [(0, 1), (0, 16), (5, 3), (13, 22), (31, 1), (7, 41)])
def test_kv_append_round_trip(start, n):
    rng = np.random.default_rng(start * 100 + n)
    bs, H, D = 8, 2, 4
    kp = rng.standard_normal((12, bs, H, D)); vp = rng.standard_normal((12, bs, H, D))
    kp0, vp0 = kp.copy(), vp.copy()
    table = np.array([9, 2, 11, 0, 5, 7, 1], np.int32)  # scattered pages
    k = rng.standard_normal((1, n, H, D)); v = rng.standard_normal((1, n, H, D))
    ok.kv_append(kp, vp, table[None], k, v, [start])
    np.testing.assert_array_equal(gather_tokens(kp, table, bs, start, n), k[0])
    np.testing.assert_array_equal(gather_tokens(vp, table, bs, start, n), v[0])
    # every slot outside the written positions is untouched
    touched = np.zeros(kp.shape[:2], bool)
    for p in range(start, start + n):
        touched[table[p // bs], p % bs] = True
    np.testing.assert_array_equal(kp[~touched], kp0[~touched])
    np.testing.assert_array_equal(vp[~touched], vp0[~touched])


def test_kv_append_batched_ragged():
    rng = np.random.default_rng(41)
    bs, H, D = 4, 3, 2
    kp = np.zeros((10, bs, H, D)); vp = np.zeros((10, bs, H, D))
    tables = np.array([[1, 4, 7], [0, 2, -1], [9, 8, 6]], np.int32)
    k = rng.standard_normal((3, 5, H, D)); v = rng.standard_normal((3, 5, H, D))
    starts, counts = [2, 0, 7], [5, 3, 5]
    ok.kv_append(kp, vp, tables, k, v, starts, counts)
    for b in range(3):
        got = gather_tokens(kp, tables[b], bs, starts[b], counts[b])
        np.testing.assert_array_equal(got, k[b, :counts[b]])
    # sequence 1 appends 3 of its 5 rows (positions 0..2 -> page 0, slots 0..2):
    # its slot 3 and its second page stay empty
    assert not kp[2].any() and not kp[0, 3].any()


def test_kv_append_errors():
    kp = np.zeros((4, 4, 1, 2)); vp = np.zeros_like(kp)
    x = np.ones((1, 3, 1, 2))
    with pytest.raises(ValueError):
        ok.kv_append(kp, vp, np.array([[0, 1]], np.int32), x, x, [-1])
    with pytest.raises(RuntimeError):
        ok.kv_append(kp, vp, np.array([[0, 1]], np.int32), x, x, [6])  # positions 6..8
    with pytest.raises(ValueError):
        ok.kv_append(kp, vp, np.array([[0, 9]], np.int32), x, x, [3])  # page 9 of 4
    # the reference writes the chunk before the failing block
    kp[:] = 0
    with pytest.raises(RuntimeError):
        ok.kv_append(kp, vp, np.array([[2, 1]], np.int32), np.ones((1, 3, 1, 2)), x, [6])
    assert kp[1, 2:].all() and not kp[2].any()


# ---- RoPE (oracle/rope.py) ---------------------------------------------------------

def test_rope_cache_kats():
    # position 0: cos 1, sin 0; dim 0 rotates at 1 rad per position; the last
    # pair at base**(-(half-1)/half)
    cos, sin = orope.precompute_rope_cache(5, 8, base=10000.0)
    assert cos.shape == (5, 4) and sin.shape == (5, 4)
    np.testing.assert_allclose(cos[0], 1.0) and np.testing.assert_allclose(sin[0], 0.0)
    np.testing.assert_allclose(cos[3, 0], math.cos(3.0), rtol=1e-6)
    np.testing.assert_allclose(sin[2, 3], math.sin(2 * 10000.0 ** (-3 / 4)), rtol=1e-5)


def test_rope_identity_norm_and_relative_position():
    rng = np.random.default_rng(50)
    D, half = 16, 8
    cos, sin = orope.precompute_rope_cache(64, D, dtype=np.float64)
    x = rng.standard_normal((1, 3, 2, D))
    np.testing.assert_allclose(orope.rope(x, cos, sin, 0)[:, :1], x[:, :1], rtol=0, atol=1e-15)
    r = orope.rope(x, cos, sin, 7)
    n_in = x[..., :half] ** 2 + x[..., half:] ** 2
    n_out = r[..., :half] ** 2 + r[..., half:] ** 2
    # (the cache is float32, as the reference's: cos^2 + sin^2 = 1 to ~1e-7)
    np.testing.assert_allclose(n_out, n_in, rtol=1e-6)
    # rope(q, m) . rope(k, n) depends only on m - n
    q = rng.standard_normal((1, 1, 1, D)); k = rng.standard_normal((1, 1, 1, D))
    dots = []
    for m, n in [(5, 2), (13, 10), (40, 37)]:
        dots.append(float(np.sum(orope.rope(q, cos, sin, m) * orope.rope(k, cos, sin, n))))
    np.testing.assert_allclose(dots, dots[0], rtol=1e-5, atol=1e-5)
    assert abs(dots[0] - float(np.sum(orope.rope(q, cos, sin, 6) * orope.rope(k, cos, sin, 2)))) > 1e-2


def _brute_rope_attention(q, k, v, scale, base, q_off, kv_off, causal, allowed=None):
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    half = D // 2

    def rot(x, pos):
        out = np.empty(D)
        for i in range(half):
            ang = pos * base ** (-i / half)
            out[i] = x[i] * math.cos(ang) - x[i + half] * math.sin(ang)
            out[i + half] = x[i] * math.sin(ang) + x[i + half] * math.cos(ang)
        return out
    o = np.zeros((B, Sq, H, D))
    for b in range(B):
        for h in range(H):
            ks = [rot(k[b, j, h], kv_off + j) for j in range(Sk)]
            for i in range(Sq):
                qi = rot(q[b, i, h], q_off + i)
                if allowed is not None:
                    js = [j for j in range(Sk) if not causal or allowed(i, j)]
                else:
                    js = [j for j in range(Sk) if not causal or kv_off + j <= q_off + i]
                if not js:
                    continue  # no visible key: zeros (fused_rope_attention.py:176-186)
                sc = [scale * float(np.dot(qi, ks[j])) for j in js]
                m = max(sc)
                w = [math.exp(x - m) for x in sc]
                for wj, j in zip(w, js):
                    o[b, i, h] += wj * v[b, j, h]
                o[b, i, h] /= sum(w)
    return o


@pytest.mark.parametrize("q_off,kv_off,causal,sq,sk", [
    (0, 0, True, 5, 5), (0, 0, False, 4, 6), (3, 0, True, 2, 5), (4, 4, True, 3, 3),
    (0, 4, True, 6, 5), (1, 9, True, 3, 4)])
def test_fused_rope_attention_vs_brute(q_off, kv_off, causal, sq, sk):
    rng = np.random.default_rng(51 + q_off + sk)
    q = rng.standard_normal((1, sq, 2, 8)); k = rng.standard_normal((1, sk, 2, 8))
    v = rng.standard_normal((1, sk, 2, 8))
    out = orope.fused_rope_attention(q, k, v, scale=0.4, rope_base=100.0, q_offset=q_off,
                                     kv_offset=kv_off, causal=causal)
    ref = _brute_rope_attention(q, k, v, 0.4, 100.0, q_off, kv_off, causal)
    # the oracle's angles are float32 (as the reference's cache): ~1e-6 agreement
    np.testing.assert_allclose(out, ref, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("q_off,kv_off,sq,sk", [(0, 0, 2, 6), (5, 0, 3, 7), (0, 0, 6, 3),
                                                  (4, 4, 3, 3)])
def test_fast_fused_rope_attention_vs_brute(q_off, kv_off, sq, sk):
    # fast_fused_rope_attention: offsets rotate only; SDPA's causal diagonal.
    rng = np.random.default_rng(53 + q_off + sk)
    q = rng.standard_normal((1, sq, 2, 8)); k = rng.standard_normal((1, sk, 2, 8))
    v = rng.standard_normal((1, sk, 2, 8))
    out = orope.fast_fused_rope_attention(q, k, v, scale=0.4, rope_base=100.0, q_offset=q_off,
                                          kv_offset=kv_off, causal=True)
    off = max(0, sk - sq)
    ref = _brute_rope_attention(q, k, v, 0.4, 100.0, q_off, kv_off, True,
                                allowed=lambda i, j: j <= i + off)
    np.testing.assert_allclose(out, ref, rtol=2e-5, atol=2e-6)


def test_fused_rope_attention_vs_sdpa():
    rng = np.random.default_rng(52)
    q = rng.standard_normal((2, 6, 3, 16)); k = rng.standard_normal((2, 9, 3, 16))
    v = rng.standard_normal((2, 9, 3, 16))
    cos, sin = orope.precompute_rope_cache(20, 16, dtype=np.float64)
    out = orope.fused_rope_attention(q, k, v, scale=0.25, cos_cache=cos, sin_cache=sin,
                                     q_offset=5, kv_offset=2, causal=True)
    qr = torch.from_numpy(orope.rope(q, cos, sin, 5)).transpose(1, 2)
    kr = torch.from_numpy(orope.rope(k, cos, sin, 2)).transpose(1, 2)
    mask = torch.tensor([[2 + j <= 5 + i for j in range(9)] for i in range(6)])
    ref = F.scaled_dot_product_attention(qr, kr, torch.from_numpy(v).transpose(1, 2),
                                         attn_mask=mask, scale=0.25).transpose(1, 2).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)


def test_block_table_kats():
    # tests/cache/test_paged_attention.py:311-333
    t = op.create_block_table_from_lengths(np.array([16, 32, 48]), 16)
    assert t.shape == (3, 3) and t[0, 0] == 0 and t[0, 1] == -1
    np.testing.assert_array_equal(t, [[0, -1, -1], [1, 2, -1], [3, 4, 5]])
    t = op.create_block_table_from_lengths(np.array([10, 25]), 16)
    assert t.shape == (2, 2) and t[0, 1] == -1


def test_alibi_slopes_kat():
    # docstring of mlx_primitives/cache/paged_attention.py:33-35: 8 heads -> 2^-1 .. 2^-8
    np.testing.assert_allclose(op.get_alibi_slopes(8), [2.0 ** -(i + 1) for i in range(8)])


# ---- torch SDPA (library routine) ------------------------------------------------

@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("layout", ["BSHD", "BHSD"])
def test_flash_vs_sdpa(causal, layout):
    q, k, v = (rnd((2, 47, 3, 16), s) for s in (40, 41, 42))
    mask = causal_mask(47, 47) if causal else None
    ref = sdpa(q, k, v, 0.25, mask)
    if layout == "BHSD":
        t = lambda x: np.ascontiguousarray(x.transpose(0, 2, 1, 3))
        out = oa.flash_attention(t(q), t(k), t(v), 0.25, causal, layout="BHSD").transpose(0, 2, 1, 3)
        tol = 1e-12
    else:
        out = oa.flash_attention(q, k, v, 0.25, causal, block_q=16, block_kv=8)
        tol = 2e-6  # the tiled path's 1e-6 epsilon
    np.testing.assert_allclose(out, ref, rtol=tol, atol=tol)


@pytest.mark.parametrize("causal", [True, False])
def test_window_vs_sdpa(causal):
    q, k, v = (rnd((1, 70, 2, 8), s) for s in (43, 44, 45))
    out = oa.sliding_window_attention(q, k, v, 20, scale=0.3, causal=causal)
    ref = sdpa(q, k, v, 0.3, window_mask(70, 20, causal))
    np.testing.assert_allclose(out, ref, rtol=2e-6, atol=2e-6)


def test_chunked_vs_sdpa():
    q = rnd((1, 33, 2, 8), 46); k = rnd((1, 300, 2, 8), 47); v = rnd((1, 300, 2, 8), 48)
    out = oa.chunked_cross_attention(q, k, v, chunk_size=64, scale=0.4)
    np.testing.assert_allclose(out, sdpa(q, k, v, 0.4), rtol=2e-6, atol=2e-6)


# ---- invariants ------------------------------------------------------------------

def test_block_size_independence():
    q, k, v = (rnd((2, 64, 2, 16), s) for s in (50, 51, 52))
    outs = [oa.tiled_flash_attention(q, k, v, 0.25, True, b, b) for b in (8, 16, 32, 64)]
    for o in outs[1:]:
        np.testing.assert_allclose(o, outs[0], rtol=1e-12, atol=1e-12)


def test_chunk_size_independence():
    q = rnd((2, 16, 2, 8), 53); k = rnd((2, 128, 2, 8), 54); v = rnd((2, 128, 2, 8), 55)
    outs = [oa.chunked_cross_attention_impl(q, k, v, c, 0.3, False) for c in (8, 16, 32, 64, 128)]
    for o in outs[1:]:
        np.testing.assert_allclose(o, outs[0], rtol=1e-12, atol=1e-12)


def test_merge_associative_and_commutative():
    q = rnd((1, 4, 2, 8), 56); k = rnd((1, 24, 2, 8), 57); v = rnd((1, 24, 2, 8), 58)
    parts = [oa.compute_chunk_attention(q, k[:, i:i + 8], v[:, i:i + 8], 0.5) for i in (0, 8, 16)]
    a = oa.online_softmax_merge(*oa.online_softmax_merge(*parts[0], *parts[1]), *parts[2])
    b = oa.online_softmax_merge(*parts[0], *oa.online_softmax_merge(*parts[1], *parts[2]))
    c = oa.online_softmax_merge(*parts[2], *oa.online_softmax_merge(*parts[1], *parts[0]))
    for x in (b, c):
        np.testing.assert_allclose(x[0] / x[2][..., None], a[0] / a[2][..., None], rtol=1e-12)


@pytest.mark.parametrize("mult", [10.0, 0.001])
def test_no_nan_at_extreme_scales(mult):
    # tests/attention/test_flash.py:163-211
    q, k = rnd((1, 32, 4, 64), 59) * mult, rnd((1, 32, 4, 64), 60) * mult
    v = rnd((1, 32, 4, 64), 61)
    out = oa.flash_attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32))
    assert np.isfinite(out).all()


# ---- gradients (oracle/attention_grad.py) --------------------------------------------

def _autograd_grads(q, k, v, dout, scale, allowed):
    """float64 torch autograd of softmax attention; BSHD numpy in, BSHD numpy out.
    allowed: (Sq, Sk) bool. K/V heads are expanded with repeat_interleave."""
    qt, kt, vt = (torch.from_numpy(x).requires_grad_(True) for x in (q, k, v))
    g = q.shape[2] // k.shape[2]
    qh = qt.transpose(1, 2)
    kh = kt.repeat_interleave(g, dim=2).transpose(1, 2)
    vh = vt.repeat_interleave(g, dim=2).transpose(1, 2)
    s = scale * (qh @ kh.transpose(-1, -2))
    s = s.masked_fill(~torch.from_numpy(allowed), float("-inf"))
    o = torch.softmax(s, dim=-1) @ vh
    (o.transpose(1, 2) * torch.from_numpy(dout)).sum().backward()
    return qt.grad.numpy(), kt.grad.numpy(), vt.grad.numpy()


@pytest.mark.parametrize("causal,wl,wr", [(False, -1, -1), (True, -1, -1), (True, 5, -1),
                                          (False, 4, 2), (False, -1, 3)])
@pytest.mark.parametrize("H,H_kv", [(2, 2), (4, 2), (3, 1)])
@pytest.mark.parametrize("Sq,Sk", [(9, 9), (6, 11), (11, 6)])
def test_grad_vs_autograd(causal, wl, wr, H, H_kv, Sq, Sk):
    q, k, v = rnd((2, Sq, H, 8), 1), rnd((2, Sk, H_kv, 8), 2), rnd((2, Sk, H_kv, 8), 3)
    dout = rnd((2, Sq, H, 8), 4)
    i, j = np.arange(Sq)[:, None], np.arange(Sk)[None, :]
    allowed = np.ones((Sq, Sk), bool)
    if causal:
        allowed &= j <= i
    if wl >= 0:
        allowed &= i - j <= wl
    if wr >= 0 and not causal:
        allowed &= j - i <= wr
    if not allowed.any(axis=1).all():
        pytest.skip("rows without keys have no softmax gradient in torch")
    got = oag.attention_grad(q, k, v, dout, 0.37, causal, wl, wr, layout="BSHD", eps=0.0)
    want = _autograd_grads(q, k, v, dout, 0.37, allowed)
    for a, b in zip(got, want):
        np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_grad_vs_sdpa_backward(causal):
    # tests/parity/pytorch/test_attention_parity.py:107-163: loss = sum(out)
    q, k, v = (rnd((2, 64, 4, 32), s) for s in (5, 6, 7))
    dout = np.ones_like(q)
    ts = [torch.from_numpy(x).transpose(1, 2).requires_grad_(True) for x in (q, k, v)]
    F.scaled_dot_product_attention(*ts, is_causal=causal).sum().backward()
    want = [t.grad.transpose(1, 2).numpy() for t in ts]
    got = oag.attention_grad(q, k, v, dout, 1 / math.sqrt(32), causal, eps=0.0)
    for a, b in zip(got, want):
        np.testing.assert_allclose(a, b, rtol=1e-9, atol=1e-12)


def test_grad_bhsd_layout_and_eps_effect():
    q, k, v, d = (rnd((1, 7, 2, 8), s) for s in (8, 9, 10, 11))
    a = oag.attention_grad(q, k, v, d, 0.5, True)
    t = lambda x: np.swapaxes(x, 1, 2)
    b = oag.attention_grad(t(q), t(k), t(v), t(d), 0.5, True, layout="BHSD")
    c = oag.attention_grad(q, k, v, d, 0.5, True, eps=0.0)
    for x, y, z in zip(a, b, c):
        np.testing.assert_allclose(x, t(y), rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(x, z, rtol=1e-5, atol=1e-5)  # eps = 1e-6 is a tiny shift


@pytest.mark.parametrize("causal,wl", [(True, -1), (False, 2)])
def test_grad_finite_differences(causal, wl):
    # Central differences of the pinned forward (oracle.attention.attention_rows,
    # o / (l + eps) normaliser) on a tiny case: every input element perturbed.
    B, S, H, D = 1, 5, 2, 4
    q, k, v, dout = (rnd((B, S, H, D), s) for s in (12, 13, 14, 15))
    scale = 0.6

    def loss(q, k, v):
        tot = 0.0
        for h in range(H):
            o = oa.attention_rows(q[0, :, h], k[0, :, h], v[0, :, h], np.arange(S), scale,
                                  causal, window_left=wl)
            tot += float(np.sum(o * dout[0, :, h]))
        return tot

    got = oag.attention_grad(q, k, v, dout, scale, causal, wl)
    xs = [q, k, v]
    for which in range(3):
        num = np.zeros_like(xs[which])
        for idx in np.ndindex(xs[which].shape):
            plus = [x.copy() for x in xs]
            minus = [x.copy() for x in xs]
            plus[which][idx] += 1e-6
            minus[which][idx] -= 1e-6
            num[idx] = (loss(*plus) - loss(*minus)) / 2e-6
        # atol: the closed form leaves out the O(eps) dependence through the row max
        np.testing.assert_allclose(got[which], num, rtol=1e-6, atol=1e-5)


# ---- planted mistakes are caught ---------------------------------------------------

def test_pin_catches_merge_without_rescale(monkeypatch):
    def bad_merge(ao, am, al, no, nm, nl):
        gm = np.maximum(am, nm)
        return ao + no, gm, al + nl  # forgets the exp(m - M) corrections
    monkeypatch.setattr(oa, "online_softmax_merge", bad_merge)
    with pytest.raises(AssertionError):
        test_tiled_flash_vs_brute(True, 2)


def test_pin_catches_window_off_by_one(monkeypatch):
    orig = oa.windowed_chunk_attention

    def bad(q, k, v, scale, causal, q_off, kv_off, w):
        return orig(q, k, v, scale, causal, q_off, kv_off, w - 1)  # W keys instead of W+1
    monkeypatch.setattr(oa, "windowed_chunk_attention", bad)
    with pytest.raises(AssertionError):
        test_sliding_window_vs_brute(True, 3)


def test_pin_catches_transposed_causal_mask(monkeypatch):
    orig = oa.compute_chunk_attention

    def bad(q, k, v, scale, causal=False, q_offset=0, kv_offset=0):
        return orig(q, k, v, scale, causal, kv_offset, q_offset)  # swapped offsets
    monkeypatch.setattr(oa, "compute_chunk_attention", bad)
    with pytest.raises(AssertionError):
        test_tiled_flash_vs_brute(True, 3)


def test_pin_catches_append_slot_off_by_one(monkeypatch):
    orig = ok.set_block_data

    def bad(k_pool, v_pool, block_id, k, v, start_pos=0, length=None):
        return orig(k_pool, v_pool, block_id, k, v, max(start_pos - 1, 0), length)
    monkeypatch.setattr(ok, "set_block_data", bad)
    with pytest.raises(AssertionError):
        test_kv_append_round_trip(5, 3)


def test_pin_catches_prefill_alibi_sign(monkeypatch):
    orig = op.paged_attention_prefill

    def bad(q, k_pool, v_pool, tables, lens, scale, bs, causal, alibi_slopes=None):
        flipped = None if alibi_slopes is None else -alibi_slopes  # q_pos - kv_pos
        return orig(q, k_pool, v_pool, tables, lens, scale, bs, causal, flipped)
    monkeypatch.setattr(op, "paged_attention_prefill", bad)
    with pytest.raises(AssertionError):
        test_paged_prefill_vs_sdpa()
    with pytest.raises(AssertionError):
        test_paged_prefill_general_vs_brute(True, True)


def test_pin_catches_rope_sine_sign(monkeypatch):
    orig = orope.rope

    def bad(x, cos, sin, offset=0):
        return orig(x, cos, -sin, offset)  # rotates by -angle
    monkeypatch.setattr(orope, "rope", bad)
    with pytest.raises(AssertionError):
        test_fused_rope_attention_vs_brute(3, 0, True, 2, 5)


def test_pin_catches_grad_without_rowsum_term(monkeypatch):
    monkeypatch.setattr(oag, "_score_grad", lambda p, dp, dout, o: p * dp)  # drops -rowsum
    with pytest.raises(AssertionError):
        test_grad_vs_autograd(True, -1, -1, 2, 2, 9, 9)
    with pytest.raises(AssertionError):
        test_grad_finite_differences(True, -1)


def test_pin_catches_cross_dense_bottom_right(monkeypatch):
    def bad(q, k, v, scale, causal):
        qt, kt, vt = (np.transpose(x, (0, 2, 1, 3)) for x in (q, k, v))
        sc = np.matmul(qt, np.swapaxes(kt, -1, -2)) * scale
        if causal:  # diagonal aligned at the bottom right instead of the top left
            keep = oa.sdpa_causal_keep(q.shape[1], k.shape[1])
            sc = np.where(keep[None, None], sc, oa.ATTENTION_MASK_VALUE)
        return np.transpose(np.matmul(oa._softmax_last(sc), vt), (0, 2, 1, 3))
    monkeypatch.setattr(oa, "reference_cross_attention", bad)
    with pytest.raises(AssertionError):
        test_reference_cross_dense_branch_vs_brute(True, 5, 11)
    with pytest.raises(AssertionError):
        test_reference_cross_dense_branch_vs_sdpa(True, 33, 64)


def test_pin_catches_cross_dense_epsilon(monkeypatch):
    orig = oa.reference_cross_attention
    monkeypatch.setattr(oa, "reference_cross_attention",
                        lambda q, k, v, s, c: orig(q, k, v, s, c) / (1 + 1e-6))  # l + 1e-6
    with pytest.raises(AssertionError):
        test_reference_cross_dense_branch_vs_brute(False, 7, 7)


@pytest.mark.parametrize("rule", ["top_left", "unclamped"])
def test_pin_catches_sdpa_causal_alignment(monkeypatch, rule):
    def bad(sq, sk):
        off = 0 if rule == "top_left" else sk - sq  # unclamped: rows before key 0
        return np.arange(sk)[None, :] <= np.arange(sq)[:, None] + off
    monkeypatch.setattr(oa, "sdpa_causal_keep", bad)
    case = (5, 12) if rule == "top_left" else (12, 5)
    with pytest.raises(AssertionError):
        with np.errstate(invalid="ignore"):
            test_flash_default_route_vs_brute_and_sdpa(*case, "BSHD")

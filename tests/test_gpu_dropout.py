"""GPU parity of attention with dropout (mpx_attn_fwd_dropout /
mpx_attn_bwd_dropout through flash_attention, sliding_window_attention,
chunked_cross_attention and autograd) against the CPU oracle
(oracle/dropout.py) with the same seed.

  * The keep mask: with Q = 0 every visible key weighs the same and
    V[k] = one-hot(k mod D) makes output column d count the kept visible
    keys k = d (mod D): O[q, d] * n_visible(q) * (1 - p) is that count (an
    integer: float32 / float16 exactly, bfloat16 to well under 0.5 for the
    counts used), compared with the oracle's mask for every row, column,
    batch and head, on the split-KV and the single-pass forward (kept-key
    counts per residue class, every dtype). In float32, V[k] =
    2^(k // D) * one-hot(k mod D) turns each count into a bitmap of the kept
    keys, compared key by key with the oracle's mask.
  * The forward on random inputs: float32 rtol 1e-4 / atol 1e-5, 16-bit
    max-abs 2e-2 against the float64 oracle (the plain forward's bars).
  * The gradients: the plain backward's bars (tests/test_gpu_attention_bwd.py:
    elementwise float32 1e-3 / 1e-4, float16 1e-2, bfloat16 1e-1; normwise
    2e-5 / 2e-3 / 1.5e-2) scaled by 1 / (1 - p) for the kept weights' scale.
  * The API: torch.manual_seed makes the mask reproducible, the measured
    keep rate is 1 - p within 5 sigma, dropout_p = 0 or training=False is the
    plain forward bit for bit (negative dropout_p too, as in the reference),
    dropout_p >= 1 is a ValueError.
"""

import math

import numpy as np
import pytest
import torch

from mlx_primitives.attention import (chunked_cross_attention, flash_attention,
                                      sliding_window_attention)
from mlx_primitives.attention import _launch
from mlx_primitives.attention._launch import dropout_seed, run_attention
from mlx_primitives.constants import Layout
from oracle import dropout as od

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
SEED = 0x9E3779B97F4A7C15
GRAD_TOL = {torch.float32: (1e-3, 1e-4, 2e-5), torch.float16: (1e-2, 1e-2, 2e-3),
            torch.bfloat16: (1e-1, 1e-1, 1.5e-2)}


def rnd(shape, seed, dtype, mult=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * mult).to(dtype)


def visible(Sq, Sk, causal, wl=-1, wr=-1):
    qi, ki = np.arange(Sq)[:, None], np.arange(Sk)[None, :]
    vis = np.ones((Sq, Sk), dtype=bool)
    if causal:
        vis &= ki <= qi
    if wl >= 0:
        vis &= qi - ki <= wl
    if wr >= 0 and not causal:
        vis &= ki - qi <= wr
    return vis


def mask_counts(device, dtype, B, H, Sq, Sk, D, p, seed, causal, wl=-1, wr=-1):
    """(measured, expected) kept-key counts per (b, h, q, residue d)."""
    q = torch.zeros((B, Sq, H, D), dtype=dtype, device=device)
    k = rnd((B, Sk, H, D), 1, dtype).to(device)
    v = torch.zeros((B, Sk, H, D), dtype=dtype)
    v[:, torch.arange(Sk), :, torch.arange(Sk) % D] = 1.0
    v = v.to(device)
    out = run_attention(q, k, v, Layout.BSHD, 1.0, causal, wl, wr, dropout_p=p,
                        dropout_seed_value=seed)
    torch.cuda.synchronize()
    vis = visible(Sq, Sk, causal, wl, wr)
    n = vis.sum(axis=1).astype(np.float64)  # (Sq,)
    got = out.double().cpu().numpy().transpose(0, 2, 1, 3)  # (B, H, Sq, D)
    measured = got * n[None, None, :, None] * (1.0 - p)
    keep = od.keep_mask(B, H, Sq, Sk, p, seed) & vis[None, None]
    onehot = (np.arange(Sk)[:, None] % D) == np.arange(D)[None, :]
    expected = keep.astype(np.float64) @ onehot.astype(np.float64)
    return measured, expected


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_forward_keep_mask_bit_exact(device, dtype, D, causal):
    # B * H * q-tiles well below the CU count: the split-KV path and its merge.
    B, H, Sq, Sk, p = 2, 3, 200, 1024, 0.3
    measured, expected = mask_counts(device, dtype, B, H, Sq, Sk, D, p, SEED, causal)
    err = np.abs(measured - expected).max()
    assert err < 0.25, err
    assert np.array_equal(np.rint(measured), expected)


def test_forward_keep_mask_headline_size(device):
    # The headline shape (4 x 32 heads x 4096, D = 128, causal; paired q-tile
    # slots, row indices up to 2^19): kept-key counts of two whole (b, h)
    # slices against the oracle's mask.
    B, H, S, D, p, seed = 4, 32, 4096, 128, 0.1, 0xABCDEF
    q = torch.zeros((B, S, H, D), dtype=torch.bfloat16, device=device)
    k = torch.zeros((B, S, H, D), dtype=torch.bfloat16, device=device)
    v = torch.zeros((1, S, 1, D), dtype=torch.bfloat16)
    v[0, torch.arange(S), 0, torch.arange(S) % D] = 1.0
    v = v.to(device).expand(B, S, H, D)
    out = run_attention(q, k, v, Layout.BSHD, 1.0, True, dropout_p=p, dropout_seed_value=seed)
    torch.cuda.synchronize()
    n = np.arange(1, S + 1, dtype=np.float64)
    onehot = ((np.arange(S)[:, None] % D) == np.arange(D)[None, :]).astype(np.float64)
    vis = np.tril(np.ones((S, S), dtype=bool))
    for b, h in [(0, 0), (3, 31)]:
        keep = od.keep_mask_rows((b * H + h) * S, S, S, p, seed)
        expected = (keep & vis).astype(np.float64) @ onehot
        got = out[b, :, h].double().cpu().numpy() * n[:, None] * (1.0 - p)
        assert np.abs(got - expected).max() < 0.25, (b, h)


def mask_bits(device, B, H, Sq, Sk, D, p, seed, causal, wl=-1):
    """(measured, expected) per-key keep bitmaps, float32: with Q = 0 and
    V[k] = 2^(k // D) * one-hot(k mod D), output column d times
    n_visible * (1 - p) is sum over the kept visible keys k = d (mod D) of
    2^(k // D), so bit j of its integer value says whether key j * D + d was
    kept. Sk <= 16 * D keeps every value an exact float32 integer below 2^16."""
    assert Sk <= 16 * D
    q = torch.zeros((B, Sq, H, D), dtype=torch.float32, device=device)
    k = torch.zeros((B, Sk, H, D), dtype=torch.float32, device=device)
    v = torch.zeros((B, Sk, H, D), dtype=torch.float32)
    idx = torch.arange(Sk)
    # (two advanced indices around a slice: the indexed view is (Sk, B, H))
    v[:, idx, :, idx % D] = (2.0 ** (idx // D).float())[:, None, None]
    v = v.to(device)
    out = run_attention(q, k, v, Layout.BSHD, 1.0, causal, wl, -1, dropout_p=p,
                        dropout_seed_value=seed)
    torch.cuda.synchronize()
    vis = visible(Sq, Sk, causal, wl)
    n = vis.sum(axis=1).astype(np.float64)
    got = out.double().cpu().numpy().transpose(0, 2, 1, 3)  # (B, H, Sq, D)
    measured = got * n[None, None, :, None] * (1.0 - p)
    keep = od.keep_mask(B, H, Sq, Sk, p, seed) & vis[None, None]
    weight = np.where((np.arange(Sk)[:, None] % D) == np.arange(D)[None, :],
                      2.0 ** (np.arange(Sk) // D)[:, None], 0.0)
    expected = keep.astype(np.float64) @ weight
    return measured, expected


@pytest.mark.parametrize("causal,wl", [(False, -1), (True, -1), (True, 300)])
@pytest.mark.parametrize("D,Sq", [(64, 200), (128, 2048), (128, 300)])
def test_forward_keep_mask_per_key(device, causal, wl, D, Sq):
    # Every kept key identified, not only the count per residue class: a tile
    # order or pair offset error that moves a kept weight to another key of
    # the same residue changes the bitmap. Sq = 200 runs the split-KV path,
    # Sq = 2048 (16 q-tiles per head) a single pass per q-tile.
    B, H, p, seed = 2, 3, 0.3, SEED ^ (D + Sq)
    Sk = Sq if causal else 1024
    measured, expected = mask_bits(device, B, H, Sq, Sk, D, p, seed, causal, wl)
    assert np.abs(measured - expected).max() < 0.25
    assert np.array_equal(np.rint(measured), expected)


def test_dropout_refuses_graph_capture_without_seed(device, monkeypatch):
    # A seed drawn on the host at capture time would be replayed by every
    # graph launch (the same keep mask each step), so a capture needs an
    # explicit dropout seed; the check runs before any launch.
    q = torch.zeros((1, 64, 2, 64), dtype=torch.bfloat16, device=device)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    with pytest.raises(RuntimeError, match="graph capture"):
        run_attention(q, q, q, Layout.BSHD, 0.125, True, dropout_p=0.1)
    with pytest.raises(RuntimeError, match="graph capture"):
        flash_attention(q, q, q, causal=True, dropout_p=0.1)


@pytest.mark.parametrize("p", [0.9, 0.999, 1e-3])
def test_forward_keep_mask_extreme_rates(device, p):
    # High and low rates: the threshold's rounding (p * 65536) and both hash
    # halves at the ends of their range.
    measured, expected = mask_counts(device, torch.float32, 2, 2, 64, 512, 64, p, 99, False)
    assert np.array_equal(np.rint(measured), expected)
    if p > 0.5:
        assert expected.sum() < 0.2 * 2 * 2 * 64 * 512


def test_tiny_rate_keeps_everything(device):
    # p < 2^-17 rounds to threshold 0: every weight is kept, scaled by 1 / (1 - p).
    q, k, v = (rnd((2, 200, 4, 64), 60 + i, torch.float32).to(device) for i in range(3))
    p = 1e-6
    got = run_attention(q, k, v, Layout.BSHD, 0.125, True, dropout_p=p, dropout_seed_value=5)
    plain = run_attention(q, k, v, Layout.BSHD, 0.125, True)
    torch.cuda.synchronize()
    torch.testing.assert_close(got, plain / (1 - p), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_forward_keep_mask_single_pass_and_window(device, dtype):
    # Many (batch, head) rows: one pass per q-tile (no split), paired causal
    # slots on the 16-bit kernel; then a sliding window.
    B, H, Sq, Sk, D, p = 4, 64, 256, 256, 128, 0.5
    measured, expected = mask_counts(device, dtype, B, H, Sq, Sk, D, p, 77, True)
    assert np.array_equal(np.rint(measured), expected)
    assert np.abs(measured - expected).max() < 0.25
    measured, expected = mask_counts(device, dtype, 2, 4, 300, 300, 64, 0.2, 78, True, wl=37)
    assert np.array_equal(np.rint(measured), expected)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("causal", [True, False])
def test_forward_vs_oracle(device, dtype, D, causal):
    B, S, H, p = 2, 333, 4, 0.25
    q, k, v = (rnd((B, S, H, D), i, dtype) for i in range(3))
    out = run_attention(q.to(device), k.to(device), v.to(device), Layout.BSHD,
                        1 / math.sqrt(D), causal, dropout_p=p, dropout_seed_value=SEED + D)
    torch.cuda.synchronize()
    ref = od.attention_dropout(*(x.double().numpy() for x in (q, k, v)), 1 / math.sqrt(D),
                               causal, p, SEED + D)
    got = out.double().cpu().numpy()
    assert np.isfinite(got).all()
    if dtype == torch.float32:
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
    else:
        assert np.abs(got - ref).max() <= 2e-2


def check_grads(got, want, dtype, p):
    rtol, atol, nrel = GRAD_TOL[dtype]
    atol = atol / (1.0 - p)
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        assert g.dtype == dtype and tuple(g.shape) == w.shape, name
        gn = g.double().cpu().numpy()
        assert np.isfinite(gn).all(), name
        np.testing.assert_allclose(gn, w, rtol=rtol, atol=atol, err_msg=name)
        rms = np.linalg.norm(w) / math.sqrt(w.size)
        if rms > atol:
            err = np.linalg.norm(gn - w) / np.linalg.norm(w)
            assert err <= nrel, f"{name}: normwise relative error {err:.3e} > {nrel}"


@pytest.mark.parametrize("dtype,D", [(dt, d) for dt in DTYPES for d in (64, 128)] +
                         [(dt, 256) for dt in DTYPES])
@pytest.mark.parametrize("causal,wl,H_kv", [(True, -1, 4), (False, -1, 4), (True, 50, 4),
                                            (True, -1, 2)])
def test_grad_vs_oracle(device, dtype, D, causal, wl, H_kv):
    grad_vs_oracle(device, dtype, D, causal, wl, H_kv)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal,wl,H_kv", [(True, -1, 4), (True, 50, 2)])
def test_grad_vs_oracle_recompute_schedule(device, monkeypatch, dtype, causal, wl, H_kv):
    # The dropout backward at D = 128 takes the stored-dS schedule by default;
    # this runs the other one.
    monkeypatch.setattr(_launch, "BWD_STORED_DS", False)
    grad_vs_oracle(device, dtype, 128, causal, wl, H_kv)


def grad_vs_oracle(device, dtype, D, causal, wl, H_kv):
    B, Sq, Sk, H, p, seed = 2, 300, 300, 4, 0.2, SEED ^ (D * 31 + H_kv)
    scale = 1 / math.sqrt(D)
    q = rnd((B, Sq, H, D), 10, dtype)
    k = rnd((B, Sk, H_kv, D), 11, dtype)
    v = rnd((B, Sk, H_kv, D), 12, dtype)
    do = rnd((B, Sq, H, D), 13, dtype)
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    out = run_attention(qd, kd, vd, Layout.BSHD, scale, causal, wl, -1, dropout_p=p,
                        dropout_seed_value=seed)
    out.backward(do.to(device))
    torch.cuda.synchronize()
    a = lambda x: x.double().numpy()
    ref_o = od.attention_dropout(a(q), a(k), a(v), scale, causal, p, seed, wl)
    got_o = out.detach().double().cpu().numpy()
    if dtype == torch.float32:
        np.testing.assert_allclose(got_o, ref_o, rtol=1e-4, atol=1e-5)
    else:
        assert np.abs(got_o - ref_o).max() <= 2e-2
    want = od.attention_dropout_grad(a(q), a(k), a(v), a(do), scale, causal, p, seed, wl)
    check_grads((qd.grad, kd.grad, vd.grad), want, dtype, p)


def test_api_seed_reproducible_and_keep_rate(device):
    B, S, H, D, p = 2, 512, 8, 64, 0.4
    q, k, v = (rnd((B, S, H, D), 20 + i, torch.bfloat16).to(device) for i in range(3))
    torch.manual_seed(5)
    a = flash_attention(q, k, v, causal=True, dropout_p=p)
    torch.manual_seed(5)
    b = flash_attention(q, k, v, causal=True, dropout_p=p)
    torch.manual_seed(5)
    seed = dropout_seed()
    c = run_attention(q, k, v, Layout.BSHD, 1 / math.sqrt(D), True, dropout_p=p,
                      dropout_seed_value=seed)
    torch.manual_seed(6)
    d = flash_attention(q, k, v, causal=True, dropout_p=p)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(a, c)
    assert not torch.equal(a, d)
    # keep rate of the API's mask, counted through the kernel (non-causal)
    measured, expected = mask_counts(device, torch.float32, 1, 8, 64, 1024, 64, p, seed, False)
    assert np.array_equal(np.rint(measured), expected)
    kept, total = expected.sum(), 8 * 64 * 1024
    qk = 1 - od.threshold(p) / 65536
    assert abs(kept / total - qk) <= 5 * math.sqrt(qk * (1 - qk) / total)


def test_no_dropout_is_plain_forward(device):
    q, k, v = (rnd((2, 100, 4, 64), 30 + i, torch.float16).to(device) for i in range(3))
    plain = flash_attention(q, k, v, causal=True)
    assert torch.equal(flash_attention(q, k, v, causal=True, dropout_p=0.3, training=False),
                       plain)
    assert torch.equal(flash_attention(q, k, v, causal=True, dropout_p=0.0), plain)
    # BHSD ignores dropout, as the reference's BHSD branch
    qb, kb, vb = (x.transpose(1, 2) for x in (q, k, v))
    assert torch.equal(flash_attention(qb, kb, vb, causal=True, dropout_p=0.3, layout="BHSD"),
                       plain.transpose(1, 2))
    with pytest.raises(ValueError, match="dropout_p"):
        flash_attention(q, k, v, dropout_p=1.0)
    with pytest.raises(ValueError, match="dropout_p"):
        sliding_window_attention(q, k, v, 8, dropout_p=1.0)
    with pytest.raises(ValueError, match="dropout_p"):
        chunked_cross_attention(q, k, v, dropout_p=1.5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sliding_window_and_chunked_api(device, dtype):
    B, S, H, D, p = 2, 257, 4, 32, 0.15
    q, k, v = (rnd((B, S, H, D), 40 + i, dtype) for i in range(3))
    kl, vl = rnd((B, 700, H, D), 43, dtype), rnd((B, 700, H, D), 44, dtype)
    a = lambda x: x.double().numpy()
    scale = 1 / math.sqrt(D)
    cases = [
        (lambda: sliding_window_attention(q.to(device), k.to(device), v.to(device), 20,
                                          dropout_p=p),
         lambda s: od.attention_dropout(a(q), a(k), a(v), scale, True, p, s, 20)),
        (lambda: sliding_window_attention(q.to(device), k.to(device), v.to(device), 20,
                                          causal=False, dropout_p=p),
         lambda s: od.attention_dropout(a(q), a(k), a(v), scale, False, p, s, 20, 20)),
        (lambda: chunked_cross_attention(q.to(device), kl.to(device), vl.to(device),
                                         chunk_size=128, dropout_p=p),
         lambda s: od.attention_dropout(a(q), a(kl), a(vl), scale, False, p, s)),
        (lambda: chunked_cross_attention(q.to(device), kl.to(device), vl.to(device),
                                         causal=True, dropout_p=p),
         lambda s: od.attention_dropout(a(q), a(kl), a(vl), scale, True, p, s)),
    ]
    for i, (run, ref) in enumerate(cases):
        torch.manual_seed(100 + i)
        out = run()
        torch.manual_seed(100 + i)
        want = ref(dropout_seed())
        torch.cuda.synchronize()
        got = out.double().cpu().numpy()
        assert got.shape == want.shape
        if dtype == torch.float32:
            np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5, err_msg=str(i))
        else:
            assert np.abs(got - want).max() <= 2e-2, i


def test_chunked_grad_with_dropout(device):
    B, Sq, Sk, H, D, p = 1, 130, 400, 2, 128, 0.3
    q, k, v, do = (rnd(s, 50 + i, torch.float16) for i, s in
                   enumerate([(B, Sq, H, D), (B, Sk, H, D), (B, Sk, H, D), (B, Sq, H, D)]))
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    torch.manual_seed(9)
    out = chunked_cross_attention(qd, kd, vd, dropout_p=p)
    out.backward(do.to(device))
    torch.cuda.synchronize()
    torch.manual_seed(9)
    seed = dropout_seed()
    a = lambda x: x.double().numpy()
    want = od.attention_dropout_grad(a(q), a(k), a(v), a(do), 1 / math.sqrt(D), False, p, seed)
    check_grads((qd.grad, kd.grad, vd.grad), want, torch.float16, p)

"""Pins of the dropout oracle (oracle/dropout.py), on the CPU.

  * lowbias32 against its published inverse (hash-prospector's lowbias32_r):
    the round trip holds only if every shift and multiplier of both match, and
    the multipliers' products with the inverse's are 1 mod 2^32;
  * the keep mask: keep rate within 5 sigma of 1 - t / 65536 for the low and
    high halves of the hash (even and odd keys), no correlation between
    neighbouring keys, neighbouring rows, query heads or seeds;
  * the forward and the gradients against torch autograd in float64 through
    the reference's formula weights = softmax(scores) * keep / (1 - p),
    out = weights @ v (attention/flash.py:562-576), with the same mask and
    masks built independently here; nothing dropped equals
    oracle.attention_grad.
The last group plants mistakes in the oracle and checks a pin catches each.
"""

import numpy as np
import pytest
import torch

from oracle import attention_grad as oag
from oracle import dropout as od


def test_lowbias32_published_inverse():
    assert (0x7FEB352D * 0x1D69E2A5) & 0xFFFFFFFF == 1
    assert (0x846CA68B * 0x43021123) & 0xFFFFFFFF == 1
    rng = np.random.default_rng(0)
    x = np.concatenate([np.arange(1 << 16, dtype=np.uint32),
                        rng.integers(0, 1 << 32, 1 << 18, dtype=np.uint64).astype(np.uint32),
                        np.array([0xFFFFFFFF, 0x80000000], dtype=np.uint32)])
    y = od.lowbias32(x)
    assert np.array_equal(od.lowbias32_inverse(y), x)
    assert np.array_equal(od.lowbias32(od.lowbias32_inverse(x)), x)
    assert od.lowbias32(np.uint32(0)) == 0  # the xor-shift-multiply steps fix 0
    assert len(np.unique(y[:1 << 16])) == 1 << 16


def test_threshold():
    assert od.threshold(0.0) == 0
    assert od.threshold(0.1) == 6554
    assert od.threshold(0.5) == 32768
    assert od.threshold(0.99999) == 65535  # clamped: 1 / 65536 of keys still kept


def _corr(a, b):
    a = a.astype(np.float64).ravel() - a.mean()
    b = b.astype(np.float64).ravel() - b.mean()
    return float((a * b).mean() / np.sqrt((a * a).mean() * (b * b).mean()))


@pytest.mark.parametrize("p", [0.1, 0.5, 0.9])
def test_keep_mask_statistics(p):
    B, H, Sq, Sk = 2, 4, 256, 512
    keep = od.keep_mask(B, H, Sq, Sk, p, seed=0x0123456789ABCDEF)
    q = 1.0 - od.threshold(p) / 65536.0
    for part in (keep, keep[..., 0::2], keep[..., 1::2]):
        n = part.size
        assert abs(part.mean() - q) <= 5 * np.sqrt(q * (1 - q) / n), (p, part.mean())
    lim = 5 / np.sqrt(keep.size / 2)
    assert abs(_corr(keep[..., :-1], keep[..., 1:])) < lim      # neighbouring keys
    assert abs(_corr(keep[..., :-1, :], keep[..., 1:, :])) < lim  # neighbouring rows
    assert abs(_corr(keep[:, :-1], keep[:, 1:])) < lim          # neighbouring heads
    other = od.keep_mask(B, H, Sq, Sk, p, seed=0x0123456789ABCDEE)
    assert abs(_corr(keep, other)) < lim                        # seeds one apart
    hi_only = od.keep_mask(B, H, Sq, Sk, p, seed=0x0123456789ABCDEF + (1 << 32))
    assert abs(_corr(keep, hi_only)) < lim


def test_keep_mask_layout():
    # Row r = (b * H + h) * Sq + q: slicing a bigger problem's mask does not
    # give a smaller problem's (Sq enters the row index) but the (b, h) order
    # does: batch 1 of a 2-batch mask is rows H * Sq onward.
    keep = od.keep_mask(2, 3, 10, 9, 0.5, seed=7)
    flat = od.keep_mask(1, 6, 10, 9, 0.5, seed=7)
    assert np.array_equal(keep.reshape(6, 10, 9), flat[0])
    # an odd Sk truncates the last pair's high half
    wide = od.keep_mask(2, 3, 10, 10, 0.5, seed=7)
    assert np.array_equal(wide[..., :9], keep)
    # a row range of a bigger problem is the same slice of the whole mask
    rows = od.keep_mask_rows(1 * 3 * 10 + 2 * 10, 10, 9, 0.5, seed=7)
    assert np.array_equal(rows, keep[1, 2])


def _torch_dropout_attention(q, k, v, scale, keep, p, vis):
    # weights = softmax(scores) * keep / (1 - p); out = weights @ v, heads
    # expanded with repeat_interleave (the oracle uses np.repeat).
    g = q.shape[1] // k.shape[1]
    ke, ve = k.repeat_interleave(g, dim=1), v.repeat_interleave(g, dim=1)
    s = torch.matmul(q, ke.transpose(-1, -2)) * scale
    s = s.masked_fill(~vis, float("-inf"))
    w = torch.softmax(s, dim=-1) * keep / (1.0 - p)
    return torch.matmul(w, ve)


@pytest.mark.parametrize("causal,wl,wr", [(False, -1, -1), (True, -1, -1), (True, 3, -1),
                                          (False, 2, 4)])
@pytest.mark.parametrize("H,H_kv", [(2, 2), (4, 2)])
def test_dropout_grad_vs_autograd(causal, wl, wr, H, H_kv):
    rng = np.random.default_rng(1)
    B, Sq, Sk, D, p, seed = 2, 9, 13, 8, 0.3, 12345
    q = rng.standard_normal((B, H, Sq, D))
    k = rng.standard_normal((B, H_kv, Sk, D))
    v = rng.standard_normal((B, H_kv, Sk, D))
    do = rng.standard_normal((B, H, Sq, D))
    scale = 0.4
    keep = od.keep_mask(B, H, Sq, Sk, p, seed)
    qi, ki = np.arange(Sq)[:, None], np.arange(Sk)[None, :]
    vis = np.ones((Sq, Sk), dtype=bool)
    if causal:
        vis &= ki <= qi
    if wl >= 0:
        vis &= qi - ki <= wl
    if wr >= 0 and not causal:
        vis &= ki - qi <= wr
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    out = _torch_dropout_attention(tq, tk, tv, scale, torch.tensor(keep), p, torch.tensor(vis))
    out.backward(torch.tensor(do))
    # (eps = 0: the reference's exact softmax; the kernels' 1e-6 normaliser
    # moves values by ~1e-6 relative)
    o, _ = od.attention_dropout_fwd_bhsd(q, k, v, scale, causal, keep, p, wl, wr, eps=0.0)
    np.testing.assert_allclose(o, out.detach().numpy(), rtol=1e-10, atol=1e-12)
    got = od.attention_dropout_grad(q, k, v, do, scale, causal, p, seed, wl, wr, layout="BHSD",
                                    eps=0.0)
    for g, want in zip(got, (tq.grad, tk.grad, tv.grad)):
        np.testing.assert_allclose(g, want.numpy(), rtol=1e-10, atol=1e-12)
    # the mask really drops something and the result depends on it
    assert 0 < (~keep).sum() < keep.size
    o0, _ = od.attention_dropout_fwd_bhsd(q, k, v, scale, causal, np.ones_like(keep), p, wl, wr)
    assert np.abs(o0 - o).max() > 1e-3


def test_nothing_dropped_equals_plain_gradients():
    rng = np.random.default_rng(2)
    q, k, v, do = (rng.standard_normal((1, 11, 2, 16)) for _ in range(4))
    keep = np.ones((1, 2, 11, 11), dtype=bool)
    got = od.attention_dropout_grad(q, k, v, do, 0.25, True, 0.0, keep=keep)
    want = oag.attention_grad(q, k, v, do, 0.25, True)
    for g, w in zip(got, want):
        np.testing.assert_allclose(g, w, rtol=1e-12, atol=1e-12)
    o = od.attention_dropout(q, k, v, 0.25, True, 0.0, seed=3)
    o2, _ = oag.attention_fwd_bhsd(*(np.swapaxes(x, 1, 2) for x in (q, k, v)), 0.25, True)
    np.testing.assert_allclose(o, np.swapaxes(o2, 1, 2), rtol=1e-12, atol=1e-12)


# ---- planted mistakes ----------------------------------------------------------------


def test_pin_catches_wrong_hash_shift(monkeypatch):
    def bad(x):
        x = np.asarray(x, dtype=np.uint32).copy()
        with np.errstate(over="ignore"):
            x ^= x >> np.uint32(16)
            x *= np.uint32(0x7FEB352D)
            x ^= x >> np.uint32(13)  # 15 in the published hash
            x *= np.uint32(0x846CA68B)
            x ^= x >> np.uint32(16)
        return x
    monkeypatch.setattr(od, "lowbias32", bad)
    with pytest.raises(AssertionError):
        test_lowbias32_published_inverse()


def test_pin_catches_unscaled_kept_gradient(monkeypatch):
    orig = od.attention_dropout_grad

    def bad(q, k, v, dout, scale, causal, p, seed=None, wl=-1, wr=-1, layout="BSHD", keep=None,
            eps=0.0):
        # dP without the 1 / (1 - p) of the kept weights: p = 0 in the gradient
        if keep is None:
            B, H, Sq = (q.shape[0], q.shape[1], q.shape[2]) if layout == "BHSD" else \
                (q.shape[0], q.shape[2], q.shape[1])
            Sk = k.shape[2] if layout == "BHSD" else k.shape[1]
            keep = od.keep_mask(B, H, Sq, Sk, p, seed)
        return orig(q, k, v, dout, scale, causal, 0.0, None, wl, wr, layout, keep, eps)
    monkeypatch.setattr(od, "attention_dropout_grad", bad)
    with pytest.raises(AssertionError):
        test_dropout_grad_vs_autograd(False, -1, -1, 2, 2)


def test_pin_catches_correlated_mask(monkeypatch):
    orig = od.keep_mask
    # the same mask for every row
    monkeypatch.setattr(od, "keep_mask", lambda B, H, Sq, Sk, p, seed: np.broadcast_to(
        orig(1, 1, 1, Sk, p, seed), (B, H, Sq, Sk)))
    with pytest.raises(AssertionError):
        test_keep_mask_statistics(0.5)

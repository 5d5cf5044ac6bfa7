"""Seeded random sweep of the GPU paths against the CPU oracle.

The hand-picked cases of the per-path tests name the shapes, masks and page
sizes the kernels branch on; this sweep draws combinations from fixed seeds
(dtype, layout, head dim, batch, heads, sequence lengths, causal / window /
chunk, grouped heads, paged decode or prefill, page size, ALiBi, empty
sequences and missing pages, dropout rate and seed), so that combinations
nobody listed run too. Every case is small enough for the float64 oracle to
finish within seconds.

Tolerances, as in the per-path tests: forward and decode float32 rtol 1e-4 /
atol 1e-5 (the reference's fp32 bar, tests/attention/test_flash.py:72-74),
16-bit max-abs error <= 2e-2 against the float64 oracle on the same cast
inputs; gradients float32 rtol 1e-3 / atol 1e-4, float16 1e-2 / 1e-2,
bfloat16 1e-1 / 1e-1 elementwise (the reference's gradient bar,
tests/parity/shared/tolerance_config.py:57,363-387); with dropout the
gradients' absolute bar is divided by 1 - p (the kept weights' scale) and a
normwise relative bar is added (float32 2e-5, float16 2e-3, bfloat16 1.5e-2),
as in the dropout tests.
"""

import numpy as np
import pytest
import torch

from mlx_primitives.attention import (chunked_cross_attention, flash_attention,
                                      sliding_window_attention)
from mlx_primitives.cache import get_alibi_slopes, paged_attention
from oracle import attention as oa
from mlx_primitives.attention._launch import run_attention
from mlx_primitives.constants import Layout
from oracle import attention_grad as oag
from oracle import dropout as od
from oracle import paged as op

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
GRAD_TOL = {torch.float32: (1e-3, 1e-4), torch.float16: (1e-2, 1e-2),
            torch.bfloat16: (1e-1, 1e-1)}
GRAD_NORMWISE = {torch.float32: 2e-5, torch.float16: 2e-3, torch.bfloat16: 1.5e-2}


def rnd(shape, gen, dtype):
    return torch.randn(shape, generator=gen).to(dtype)


def check(out, ref, dtype, what):
    got = out.double().cpu().numpy()
    assert got.shape == ref.shape, what
    nan_ref = np.isnan(ref)
    assert (np.isnan(got) == nan_ref).all(), f"{what}: NaN rows differ"
    g, r = got[~nan_ref], ref[~nan_ref]
    assert np.isfinite(g).all(), what
    if dtype == torch.float32:
        np.testing.assert_allclose(g, r, rtol=1e-4, atol=1e-5, err_msg=what)
    else:
        err = float(np.abs(g - r).max()) if g.size else 0.0
        assert err <= 2e-2, f"{what}: max abs err {err}"


@pytest.mark.parametrize("seed", range(60))
def test_forward_sweep(device, seed):
    rng = np.random.default_rng(7000 + seed)
    gen = torch.Generator().manual_seed(7000 + seed)
    dtype = DTYPES[int(rng.integers(3))]
    D = int(rng.choice([32, 48, 64, 96, 128, 160, 256]))
    B, H = int(rng.integers(1, 3)), int(rng.integers(1, 5))
    kind = ("flash", "window", "chunked")[seed % 3]
    a = lambda x: x.double().numpy()
    d = lambda x: x.to(device)
    if kind == "flash":
        S = int(rng.integers(1, 700))
        causal = bool(rng.integers(2))
        layout = ("BSHD", "BHSD")[int(rng.integers(2))]
        G = int(rng.choice([1, 1, 2, 3]))  # query heads per K/V head (enable_gqa)
        shape = lambda h: (B, S, h, D) if layout == "BSHD" else (B, h, S, D)
        q = rnd(shape(H * G), gen, dtype)
        k, v = (rnd(shape(H), gen, dtype) for _ in range(2))
        out = flash_attention(d(q), d(k), d(v), causal=causal, layout=layout, enable_gqa=G > 1)
        hd = 2 if layout == "BSHD" else 1
        ke, ve = (x.repeat_interleave(G, dim=hd) for x in (k, v))
        ref = oa.flash_attention(a(q), a(ke), a(ve), causal=causal, layout=layout)
        what = f"flash {dtype} {layout} B={B} H={H * G}/{H} S={S} D={D} causal={causal}"
    elif kind == "window":
        S, W = int(rng.integers(1, 900)), int(rng.integers(0, 300))
        causal = bool(rng.integers(2))
        q, k, v = (rnd((B, S, H, D), gen, dtype) for _ in range(3))
        out = sliding_window_attention(d(q), d(k), d(v), W, causal=causal)
        ref = oa.sliding_window_attention(a(q), a(k), a(v), W, causal=causal)
        what = f"window {dtype} B={B} H={H} S={S} W={W} D={D} causal={causal}"
    else:
        Sq, Sk = int(rng.integers(1, 300)), int(rng.integers(1, 3000))
        chunk = int(rng.choice([128, 256, 1024]))
        q = rnd((B, Sq, H, D), gen, dtype)
        k, v = (rnd((B, Sk, H, D), gen, dtype) for _ in range(2))
        out = chunked_cross_attention(d(q), d(k), d(v), chunk_size=chunk)
        ref = oa.chunked_cross_attention(a(q), a(k), a(v), chunk_size=chunk)
        what = f"chunked {dtype} B={B} H={H} Sq={Sq} Sk={Sk} chunk={chunk} D={D}"
    torch.cuda.synchronize()
    check(out, ref, dtype, what)


@pytest.mark.parametrize("seed", range(60))
def test_paged_sweep(device, seed):
    rng = np.random.default_rng(8000 + seed)
    gen = torch.Generator().manual_seed(8000 + seed)
    dtype = DTYPES[int(rng.integers(3))]
    D = int(rng.choice([32, 64, 80, 128, 128, 256]))
    H_kv, G = int(rng.choice([1, 2, 4, 8])), int(rng.choice([1, 2, 3, 4, 8]))
    H = H_kv * G
    bs = int(rng.choice([8, 16, 24, 32, 64]))
    B = int(rng.integers(1, 9))
    # decode (one query token) or prefill (Sq tokens, the last Sq of each context)
    Sq = 1 if seed % 2 == 0 else int(rng.integers(2, 130))
    causal = Sq == 1 or bool(rng.integers(2))
    lens = np.maximum(rng.integers(0, 3000, size=B), Sq)
    if B > 1 and rng.integers(2):
        lens[int(rng.integers(B))] = 0  # an empty sequence: NaN row
    pages = [(int(n) + bs - 1) // bs for n in lens]
    nb = sum(pages) + 2
    perm = rng.permutation(nb)
    tables = np.full((B, max(max(pages), 1)), -1, np.int32)
    off = 0
    for b, n in enumerate(pages):
        tables[b, :n] = perm[off:off + n]
        off += n
    if rng.integers(2):
        b = int(np.argmax(pages))
        if pages[b] > 1:
            tables[b, int(rng.integers(pages[b]))] = -1  # a missing page
    q = rnd((B, Sq, H, D), gen, dtype)
    kp, vp = (rnd((nb, bs, H_kv, D), gen, dtype) for _ in range(2))
    slopes = get_alibi_slopes(H) if rng.integers(2) else None
    d = lambda x: x.to(device)
    out = paged_attention(d(q), d(kp), d(vp), d(torch.from_numpy(tables)),
                          d(torch.tensor(lens, dtype=torch.int32)), block_size=bs,
                          causal=causal, alibi_slopes=None if slopes is None else d(slopes),
                          enable_gqa=G > 1)
    torch.cuda.synchronize()
    ref = op.paged_attention(q.double().numpy(), kp.repeat_interleave(G, dim=2).double().numpy(),
                             vp.repeat_interleave(G, dim=2).double().numpy(), tables,
                             lens.astype(np.int32), block_size=bs, causal=causal,
                             alibi_slopes=None if slopes is None else slopes.double().numpy())
    check(out, ref, dtype, f"paged {dtype} Sq={Sq} causal={causal} B={B} H={H} H_kv={H_kv} "
                           f"D={D} bs={bs} "
                           f"alibi={slopes is not None} lens={lens.tolist()}")


@pytest.mark.parametrize("seed", range(24))
def test_backward_sweep(device, seed):
    rng = np.random.default_rng(9000 + seed)
    gen = torch.Generator().manual_seed(9000 + seed)
    dtype = DTYPES[int(rng.integers(3))]
    D = int(rng.choice([32, 64, 96, 128, 256]))
    B, H, S = int(rng.integers(1, 3)), int(rng.integers(1, 4)), int(rng.integers(1, 400))
    windowed = bool(rng.integers(2))
    causal = bool(rng.integers(2))
    W = int(rng.integers(1, 200))
    q, k, v, dout = (rnd((B, S, H, D), gen, dtype) for _ in range(4))
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    if windowed:
        out = sliding_window_attention(qd, kd, vd, W, causal=causal)
        wl, wr = W, (-1 if causal else W)  # (with causal the right edge is the diagonal)
    else:
        out = flash_attention(qd, kd, vd, causal=causal)
        wl, wr = -1, -1
    out.backward(dout.to(device))
    torch.cuda.synchronize()
    a = lambda x: x.double().numpy()
    want = oag.attention_grad(a(q), a(k), a(v), a(dout), 1.0 / np.sqrt(D), causal, wl, wr)
    rtol, atol = GRAD_TOL[dtype]
    what = f"grad {dtype} B={B} H={H} S={S} D={D} causal={causal} window={W if windowed else None}"
    for name, g, w in zip(("dq", "dk", "dv"), (qd.grad, kd.grad, vd.grad), want):
        gn = g.double().cpu().numpy()
        assert np.isfinite(gn).all(), f"{what} {name}"
        np.testing.assert_allclose(gn, w, rtol=rtol, atol=atol, err_msg=f"{what} {name}")


@pytest.mark.parametrize("seed", range(24))
def test_dropout_sweep(device, seed):
    # forward and gradients with dropout: the keep mask of (seed, row, key
    # pair) regenerated by the backward kernels, against the oracle's mask
    rng = np.random.default_rng(9500 + seed)
    gen = torch.Generator().manual_seed(9500 + seed)
    dtype = DTYPES[int(rng.integers(3))]
    D = int(rng.choice([32, 64, 96, 128, 256]))
    B, H_kv, G = int(rng.integers(1, 3)), int(rng.integers(1, 4)), int(rng.choice([1, 2]))
    S = int(rng.integers(1, 400))
    causal = bool(rng.integers(2))
    wl = int(rng.integers(1, 200)) if rng.integers(2) else -1
    p = float(rng.choice([0.1, 0.3, 0.6]))
    dseed = int(rng.integers(1 << 62))
    scale = 1.0 / np.sqrt(D)
    q, dout = (rnd((B, S, H_kv * G, D), gen, dtype) for _ in range(2))
    k, v = (rnd((B, S, H_kv, D), gen, dtype) for _ in range(2))
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    out = run_attention(qd, kd, vd, Layout.BSHD, scale, causal, wl, -1, dropout_p=p,
                        dropout_seed_value=dseed)
    out.backward(dout.to(device))
    torch.cuda.synchronize()
    a = lambda x: x.double().numpy()
    what = (f"dropout {dtype} B={B} H={H_kv * G}/{H_kv} S={S} D={D} causal={causal} "
            f"window={wl} p={p}")
    ref = od.attention_dropout(a(q), a(k), a(v), scale, causal, p, dseed, wl)
    check(out.detach(), ref, dtype, what)
    want = od.attention_dropout_grad(a(q), a(k), a(v), a(dout), scale, causal, p, dseed, wl)
    rtol, atol = GRAD_TOL[dtype]
    atol /= 1.0 - p
    for name, g, w in zip(("dq", "dk", "dv"), (qd.grad, kd.grad, vd.grad), want):
        gn = g.double().cpu().numpy()
        assert gn.shape == w.shape and np.isfinite(gn).all(), f"{what} {name}"
        np.testing.assert_allclose(gn, w, rtol=rtol, atol=atol, err_msg=f"{what} {name}")
        if np.linalg.norm(w) / np.sqrt(w.size) > atol:
            err = np.linalg.norm(gn - w) / np.linalg.norm(w)
            assert err <= GRAD_NORMWISE[dtype], f"{what} {name}: normwise {err:.3e}"

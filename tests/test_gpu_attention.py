"""GPU parity of flash / sliding-window / chunked attention (HIP kernels,
through the C ABI) against the CPU oracle on identical inputs.

Tolerances (written per test): float32 outputs rtol 1e-4 / atol 1e-5 (the
reference's fp32 test tolerance, tests/attention/test_flash.py:72-74);
bfloat16 / float16 max-abs error <= 2e-2 against the float64 oracle run on the
same cast inputs.
"""

import math

import numpy as np
import pytest
import torch

from mlx_primitives.attention import (
    ChunkedCrossAttention,
    FlashAttention,
    SlidingWindowAttention,
    chunked_cross_attention,
    flash_attention,
    sliding_window_attention,
)
from oracle import attention as oa
import workloads as wl

pytestmark = pytest.mark.gpu

F32_RTOL, F32_ATOL = 1e-4, 1e-5
LOWP_MAXABS = 2e-2
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def inputs(shapes, dtype, seed, device, mult=1.0):
    g = torch.Generator().manual_seed(seed)
    xs = [torch.randn(s, generator=g) for s in shapes]
    xs[0] = xs[0] * mult
    xs[1] = xs[1] * mult
    cast = [x.to(dtype) for x in xs]
    return [x.to(device) for x in cast], [x.double().numpy() for x in cast]


def check(out_gpu, ref, dtype):
    got = out_gpu.double().cpu().numpy()
    assert got.shape == ref.shape
    assert np.isfinite(got).all()
    if dtype == torch.float32:
        np.testing.assert_allclose(got, ref, rtol=F32_RTOL, atol=F32_ATOL)
    else:
        err = np.abs(got - ref).max()
        assert err <= LOWP_MAXABS, f"max abs err {err}"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("layout", ["BSHD", "BHSD"])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_flash_parity(device, dtype, layout, causal, D):
    B, S, H = 2, 300, 3
    shape = (B, S, H, D) if layout == "BSHD" else (B, H, S, D)
    (q, k, v), (qn, kn, vn) = inputs([shape] * 3, dtype, 1000 + D, device)
    out = flash_attention(q, k, v, causal=causal, layout=layout)
    assert out.dtype == dtype and out.shape == q.shape
    ref = oa.flash_attention(qn, kn, vn, causal=causal, layout=layout)
    check(out, ref, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("layout", ["BSHD", "BHSD"])
@pytest.mark.parametrize("Sq,Sk,D", [(1, 300, 64), (77, 300, 128), (300, 77, 64),
                                     (5, 5000, 128), (257, 513, 32), (1, 1, 64)])
def test_flash_causal_alignment(device, dtype, layout, Sq, Sk, D):
    # causal=True with Sq != Sk follows the reference's default (SDPA) route:
    # key j visible to query i iff j <= i + max(0, Sk - Sq) -- a decode step
    # over a cache sees every key, Sq > Sk is top-left aligned.
    B, H = 2, 3
    qs = (B, Sq, H, D) if layout == "BSHD" else (B, H, Sq, D)
    ks = (B, Sk, H, D) if layout == "BSHD" else (B, H, Sk, D)
    (q, k, v), (qn, kn, vn) = inputs([qs, ks, ks], dtype, 7 * Sq + Sk, device)
    out = flash_attention(q, k, v, causal=True, layout=layout)
    assert out.dtype == dtype and out.shape == q.shape
    check(out, oa.flash_attention_default_route(qn, kn, vn, causal=True, layout=layout), dtype)


@pytest.mark.parametrize("S", [1, 2, 31, 47, 64, 127, 129, 192, 320, 513])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_flash_ragged_lengths(device, S, dtype):
    # 192 and 320 end on a 64-key half of a 128-key tile.
    (q, k, v), (qn, kn, vn) = inputs([(1, S, 2, 64)] * 3, dtype, S, device)
    check(flash_attention(q, k, v, causal=True), oa.flash_attention(qn, kn, vn, causal=True), dtype)


@pytest.mark.parametrize("S", [192, 320])
@pytest.mark.parametrize("causal", [True, False])
def test_flash_half_tile_d128(device, S, causal):
    """D = 128 (two 64 KB stages of 128-key tiles) ending on a 64-key half tile."""
    (q, k, v), (qn, kn, vn) = inputs([(1, S, 2, 128)] * 3, torch.bfloat16, S + 7, device)
    check(flash_attention(q, k, v, causal=causal), oa.flash_attention(qn, kn, vn, causal=causal),
          torch.bfloat16)


@pytest.mark.parametrize("S,D", [(1100, 64), (1100, 128), (1536, 64), (1280, 32)])
def test_flash_paired_causal_slots(device, S, D):
    # 96 (batch, head) pairs x >= 3 q-tile slots: the causal launch pairs q-tile i
    # with q-tile n-1-i in one workgroup. S=1100 / 1280 give 5 q-tiles (the middle
    # slot runs a single q-tile; 1100 also has a ragged last tile), 1536 gives 6.
    (q, k, v), (qn, kn, vn) = inputs([(2, 48, S, D)] * 3, torch.bfloat16, S + D, device)
    out = flash_attention(q, k, v, causal=True, layout="BHSD")
    sel = [0, 13, 47]
    ref = oa.flash_attention(qn[:, sel], kn[:, sel], vn[:, sel], causal=True, layout="BHSD")
    check(out[:, sel], ref, torch.bfloat16)


@pytest.mark.parametrize("BH,S,D", [(136, 768, 128), (96, 1536, 64)])
def test_flash_paired_single_tail_every_head(device, BH, S, D):
    # B * H divisible by the 8 XCDs: each XCD's slice of (batch, head)s runs
    # paired slots first, then the q-tiles of its last heads one per workgroup
    # (768: 3 q-tiles, 2 slots, 16 of 17 heads per XCD single; 1536: 6
    # q-tiles, 3 slots, 11 of 12). Every head is checked.
    (q, k, v), (qn, kn, vn) = inputs([(1, BH, S, D)] * 3, torch.bfloat16, BH + S, device)
    out = flash_attention(q, k, v, causal=True, layout="BHSD")
    check(out, oa.flash_attention(qn, kn, vn, causal=True, layout="BHSD"), torch.bfloat16)


@pytest.mark.parametrize("D", [1, 8, 16, 40, 80, 96])
def test_flash_padded_head_dims(device, D):
    (q, k, v), (qn, kn, vn) = inputs([(2, 70, 2, D)] * 3, torch.float32, D, device)
    out = flash_attention(q, k, v, causal=True)
    check(out, oa.flash_attention(qn, kn, vn, causal=True), torch.float32)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("layout", ["BSHD", "BHSD"])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [160, 256])
def test_flash_head_dims_above_128(device, dtype, layout, causal, D):
    # Head dims 129 .. 256 run on the D = 256 kernels (inputs zero-padded);
    # B * H * q-tiles below the CU count: the split-KV path.
    B, S, H = 2, 300, 3
    shape = (B, S, H, D) if layout == "BSHD" else (B, H, S, D)
    (q, k, v), (qn, kn, vn) = inputs([shape] * 3, dtype, D + S, device)
    out = flash_attention(q, k, v, causal=causal, layout=layout)
    check(out, oa.flash_attention(qn, kn, vn, causal=causal, layout=layout), dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_flash_head_dim_256_single_pass_paired(device, dtype):
    # 4 x 64 (batch, head) pairs x 4 q-tiles: no split; the 16-bit causal
    # launch pairs q-tiles.
    (q, k, v), (qn, kn, vn) = inputs([(4, 64, 512, 256)] * 3, dtype, 5, device)
    out = flash_attention(q, k, v, causal=True, layout="BHSD")
    sel = [0, 31, 63]
    ref = oa.flash_attention(qn[:1, sel], kn[:1, sel], vn[:1, sel], causal=True, layout="BHSD")
    check(out[:1, sel], ref, dtype)


def test_head_dim_256_window_and_chunked(device):
    (q, k, v), (qn, kn, vn) = inputs([(2, 333, 2, 256)] * 3, torch.float16, 17, device)
    check(sliding_window_attention(q, k, v, 40),
          oa.sliding_window_attention(qn, kn, vn, 40, causal=True), torch.float16)
    check(sliding_window_attention(q, k, v, 40, causal=False),
          oa.sliding_window_attention(qn, kn, vn, 40, causal=False), torch.float16)
    (q, k, v), (qn, kn, vn) = inputs([(1, 64, 2, 200), (1, 3000, 2, 200), (1, 3000, 2, 200)],
                                     torch.bfloat16, 18, device)
    check(chunked_cross_attention(q, k, v, chunk_size=512),
          oa.chunked_cross_attention(qn, kn, vn, chunk_size=512), torch.bfloat16)


def test_head_dim_limits(device):
    x = torch.zeros(1, 8, 1, 264, device=device)
    with pytest.raises(NotImplementedError, match="256"):
        flash_attention(x, x, x)
    y = torch.zeros(1, 8, 1, 264, device=device, requires_grad=True)
    with pytest.raises(NotImplementedError, match="256"):
        flash_attention(y, y, y)
    with pytest.raises(NotImplementedError, match="256"):
        flash_attention(x, x, x, dropout_p=0.1)
    from mlx_primitives.cache import paged_attention
    q = torch.zeros(2, 1, 2, 264, device=device)
    pool = torch.zeros(4, 16, 2, 264, device=device)
    with pytest.raises(NotImplementedError, match="paged attention.*256"):
        paged_attention(q, pool, pool, torch.zeros(2, 1, dtype=torch.int32, device=device),
                        torch.ones(2, dtype=torch.int32, device=device))


@pytest.mark.parametrize("scale", [0.05, 1.0, -0.3])
def test_flash_explicit_scale(device, scale):
    (q, k, v), (qn, kn, vn) = inputs([(1, 100, 2, 64)] * 3, torch.float32, 7, device)
    check(flash_attention(q, k, v, scale=scale), oa.flash_attention(qn, kn, vn, scale=scale),
          torch.float32)


@pytest.mark.parametrize("mult", [10.0, 0.001])
def test_flash_extreme_input_scales(device, mult):
    # tests/attention/test_flash.py:163-211: no NaN/Inf at x10 / x0.001
    # At x10 the logits reach ~1e2: fp32 rounding of q.k (~1e-7 * |q||k|) alone moves
    # the weights by ~1e-4 relative, so the comparison with the float64 oracle uses a
    # 1e-3 relative bound there; the reference checks only finiteness.
    (q, k, v), (qn, kn, vn) = inputs([(1, 64, 4, 64)] * 3, torch.float32, 8, device, mult)
    out = flash_attention(q, k, v, causal=True)
    got = out.double().cpu().numpy()
    assert np.isfinite(got).all()
    rtol = 1e-3 if mult > 1 else F32_RTOL
    np.testing.assert_allclose(got, oa.flash_attention(qn, kn, vn, causal=True), rtol=rtol,
                               atol=F32_ATOL)


def test_flash_non_contiguous_inputs(device):
    (q, k, v), (qn, kn, vn) = inputs([(2, 3, 96, 64)] * 3, torch.bfloat16, 9, device)
    qt, kt, vt = (x.transpose(1, 2) for x in (q, k, v))  # BSHD views of BHSD storage
    out = flash_attention(qt, kt, vt, causal=True)
    ref = oa.flash_attention(*(np.ascontiguousarray(x.transpose(0, 2, 1, 3)) for x in (qn, kn, vn)),
                             causal=True)
    check(out, ref, torch.bfloat16)


def test_flash_kats(device):
    # tests/reference.py:453-468 (attention_identity) and test_flash.py:217-230
    q = torch.ones(1, 4, 1, 1, device=device)
    v = torch.tensor([1.0, 2.0, 3.0, 4.0], device=device).reshape(1, 4, 1, 1)
    out = flash_attention(q, q, v, scale=1.0, causal=True)
    np.testing.assert_allclose(out.cpu().numpy().ravel(), [1.0, 1.5, 2.0, 2.5], rtol=1e-5)
    (q, k, v), _ = inputs([(2, 1, 4, 64)] * 3, torch.float32, 10, device)
    np.testing.assert_allclose(flash_attention(q, k, v).cpu().numpy(), v.cpu().numpy(),
                               rtol=1e-5, atol=1e-6)


def test_flash_deterministic(device):
    (q, k, v), _ = inputs([(2, 512, 4, 128)] * 3, torch.bfloat16, 11, device)
    a = flash_attention(q, k, v)
    b = flash_attention(q, k, v)
    assert torch.equal(a, b)


def test_flash_module(device):
    (q, k, v), (qn, kn, vn) = inputs([(2, 64, 8, 64)] * 3, torch.float32, 12, device)
    check(FlashAttention(8, 64, causal=False)(q, k, v),
          oa.flash_attention(qn, kn, vn, causal=False), torch.float32)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("W", [0, 1, 7, 64, 100, 400])
def test_sliding_window_parity(device, dtype, causal, W):
    (q, k, v), (qn, kn, vn) = inputs([(2, 333, 2, 64)] * 3, dtype, 2000 + W, device)
    out = sliding_window_attention(q, k, v, window_size=W, causal=causal)
    ref = oa.sliding_window_attention(qn, kn, vn, W, causal=causal)
    check(out, ref, dtype)


def test_sliding_window_full_equals_causal(device):
    (q, k, v), _ = inputs([(2, 200, 2, 128)] * 3, torch.bfloat16, 13, device)
    a = sliding_window_attention(q, k, v, window_size=200, causal=True)
    b = flash_attention(q, k, v, causal=True)
    assert (a.float() - b.float()).abs().max().item() < 1e-2


def test_sliding_window_module(device):
    (q, k, v), (qn, kn, vn) = inputs([(1, 128, 8, 64)] * 3, torch.float32, 14, device)
    check(SlidingWindowAttention(8, 64, 32)(q, k, v),
          oa.sliding_window_attention(qn, kn, vn, 32), torch.float32)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("Sq,Skv", [(16, 32), (1, 256), (64, 5000), (200, 20000)])
@pytest.mark.parametrize("causal", [False, True])
def test_chunked_parity(device, dtype, Sq, Skv, causal):
    (q, k, v), (qn, kn, vn) = inputs([(1, Sq, 2, 64), (1, Skv, 2, 64), (1, Skv, 2, 64)], dtype,
                                     Sq + Skv, device)
    out = chunked_cross_attention(q, k, v, chunk_size=1024, causal=causal)
    ref = oa.chunked_cross_attention(qn, kn, vn, chunk_size=1024, causal=causal)
    check(out, ref, dtype)


def test_chunked_module(device):
    (q, k, v), (qn, kn, vn) = inputs([(1, 32, 4, 64), (1, 4096, 4, 64), (1, 4096, 4, 64)],
                                     torch.float32, 15, device)
    check(ChunkedCrossAttention(4, 64)(q, k, v), oa.chunked_cross_attention(qn, kn, vn),
          torch.float32)


# ---- full BASELINE configurations -------------------------------------------------

def _sample_rows_check(out, q, k, v, cfg, rows_per_head=24, heads=4, seed=0, **mask):
    """Exact oracle on sampled (b, h, q) rows of a full-size run."""
    rng = np.random.default_rng(seed)
    bhsd = cfg.get("layout") == "BHSD"
    B = q.shape[0]
    H = q.shape[1] if bhsd else q.shape[2]
    Sq = q.shape[2] if bhsd else q.shape[1]
    scale = 1.0 / math.sqrt(q.shape[-1])
    worst = 0.0
    for _ in range(heads):
        b, h = int(rng.integers(B)), int(rng.integers(H))
        sel = lambda x: (x[b, h] if bhsd else x[b, :, h]).double().cpu().numpy()
        rows = np.unique(np.concatenate([[0, Sq - 1], rng.integers(0, Sq, rows_per_head)]))
        ref = oa.attention_rows(sel(q)[rows], sel(k), sel(v), rows, scale, **mask)
        got = sel(out)[rows]
        worst = max(worst, float(np.abs(got - ref).max()))
    return worst


def _slice_check(out, q, k, v, cfg, bh, block=1024, **mask):
    """Exact oracle on every query row of the (batch, head) slices in bh."""
    bhsd = cfg.get("layout") == "BHSD"
    Sq = q.shape[2] if bhsd else q.shape[1]
    scale = 1.0 / math.sqrt(q.shape[-1])
    worst = 0.0
    for b, h in bh:
        sel = lambda x: (x[b, h] if bhsd else x[b, :, h]).double().cpu().numpy()
        qs, ks, vs, os_ = sel(q), sel(k), sel(v), sel(out)
        for r0 in range(0, Sq, block):
            rows = np.arange(r0, min(Sq, r0 + block))
            ref = oa.attention_rows(qs[rows], ks, vs, rows, scale, **mask)
            worst = max(worst, float(np.abs(os_[rows] - ref).max()))
    return worst


def test_config1_flash_fp32_full(device):
    cfg = wl.CONFIGS["flash_fp32_bshd"]
    q, k, v = wl.make_qkv(cfg)
    out = flash_attention(q.to(device), k.to(device), v.to(device), causal=True)
    ref = oa.flash_attention(*(x.double().numpy() for x in (q, k, v)), causal=True)
    np.testing.assert_allclose(out.double().cpu().numpy(), ref, rtol=F32_RTOL, atol=F32_ATOL)


def test_config2_flash_bf16_full(device):
    cfg = wl.CONFIGS["flash_bf16_bhsd"]
    q, k, v = wl.make_qkv(cfg, device=device)
    out = flash_attention(q, k, v, causal=True, layout="BHSD")
    assert torch.isfinite(out.float()).all()
    assert _sample_rows_check(out, q, k, v, cfg, causal=True) <= LOWP_MAXABS
    # two whole (batch, head) slices: the first and the last
    assert _slice_check(out, q, k, v, cfg, [(0, 0), (3, 31)], causal=True) <= LOWP_MAXABS
    assert torch.equal(out, flash_attention(q, k, v, causal=True, layout="BHSD"))


def test_config3_window_bf16_full(device):
    cfg = wl.CONFIGS["window_bf16_bshd"]
    q, k, v = wl.make_qkv(cfg, device=device)
    out = SlidingWindowAttention(cfg["H"], cfg["D"], cfg["window"], causal=True)(q, k, v)
    assert torch.isfinite(out.float()).all()
    err = _sample_rows_check(out, q, k, v, cfg, causal=True, window_left=cfg["window"])
    assert err <= LOWP_MAXABS
    err = _slice_check(out, q, k, v, cfg, [(1, 17)], causal=True, window_left=cfg["window"])
    assert err <= LOWP_MAXABS


def test_config5_chunked_bf16_full(device):
    cfg = wl.CONFIGS["chunked_bf16"]
    q, k, v = wl.make_qkv(cfg, device=device)
    out = ChunkedCrossAttention(cfg["H"], cfg["D"], cfg["chunk_size"])(q, k, v)
    assert torch.isfinite(out.float()).all()
    assert _sample_rows_check(out, q, k, v, cfg, causal=False) <= LOWP_MAXABS
    assert _slice_check(out, q, k, v, cfg, [(0, 0), (0, 15)], causal=False) <= LOWP_MAXABS

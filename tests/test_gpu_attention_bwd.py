"""GPU parity of the attention backward: gradients through flash_attention,
sliding_window_attention and chunked_cross_attention (autograd -> mpx_attn_bwd)
against the float64 oracle gradients (oracle/attention_grad.py) on the same
float32 / float16 / bfloat16 inputs and output cotangent.

Tolerances, per gradient tensor:
  * elementwise, the reference's gradient bar (ten times its forward bar,
    tests/parity/shared/tolerance_config.py:57,363-387): float32 rtol 1e-3 /
    atol 1e-4, float16 rtol = atol = 1e-2, bfloat16 rtol = atol = 1e-1;
  * normwise, ||g - ref|| / ||ref|| <= 2e-5 (float32), 2e-3 (float16) and
    1.5e-2 (bfloat16): a few units of the dtype's rounding (2^-24 accumulated
    over ~S terms, 2^-11 and 2^-8), which the 16-bit kernels incur by rounding
    P and dS to the MFMA input type and the result to dtype;
    checked where the reference's RMS exceeds the elementwise atol (a gradient
    that vanishes, like dq with one visible key, is pure rounding noise).
"""

import math

import numpy as np
import pytest
import torch

from mlx_primitives.attention import (chunked_cross_attention, flash_attention,
                                      sliding_window_attention)
from mlx_primitives.attention import _launch
from oracle import attention_grad as oag

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (1e-3, 1e-4, 2e-5), torch.float16: (1e-2, 1e-2, 2e-3),
       torch.bfloat16: (1e-1, 1e-1, 1.5e-2)}
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def rnd(shape, seed, dtype, mult=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * mult).to(dtype)


def run_grads(fn, device, q, k, v, dout):
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    out = fn(qd, kd, vd)
    out.backward(dout.to(device))
    torch.cuda.synchronize()
    return out, qd.grad, kd.grad, vd.grad


def check_grads(got, q, k, v, dout, dtype, scale, causal, wl=-1, wr=-1, layout="BSHD"):
    a = lambda x: x.double().numpy()
    want = oag.attention_grad(a(q), a(k), a(v), a(dout), scale, causal, wl, wr, layout=layout)
    rtol, atol, nrel = TOL[dtype]
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        assert g.dtype == dtype and tuple(g.shape) == w.shape, name
        gn = g.double().cpu().numpy()
        assert np.isfinite(gn).all(), name
        np.testing.assert_allclose(gn, w, rtol=rtol, atol=atol, err_msg=name)
        rms = np.linalg.norm(w) / math.sqrt(w.size)
        if rms > atol:  # below the absolute floor (e.g. one visible key: dq ~ 0) atol rules
            err = np.linalg.norm(gn - w) / np.linalg.norm(w)
            print(f"{name} normwise rel err {err:.2e}")
            assert err <= nrel, f"{name}: normwise relative error {err:.3e} > {nrel}"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("layout", ["BSHD", "BHSD"])
@pytest.mark.parametrize("D", [32, 64, 80, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_flash_grad(device, dtype, layout, D, causal):
    B, H, S = 2, 3, 300
    shape = (B, S, H, D) if layout == "BSHD" else (B, H, S, D)
    q, k, v, d = (rnd(shape, D + i, dtype) for i in range(4))
    scale = 1 / math.sqrt(D)
    fn = lambda q, k, v: flash_attention(q, k, v, causal=causal, layout=layout)
    out, *g = run_grads(fn, device, q, k, v, d)
    check_grads(g, q, k, v, d, dtype, scale, causal, layout=layout)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("layout", ["BSHD", "BHSD"])
@pytest.mark.parametrize("D", [160, 256])
@pytest.mark.parametrize("causal", [True, False])
def test_flash_grad_head_dims_above_128(device, dtype, layout, D, causal):
    # Head dims 129 .. 256: the D = 256 backward kernels (16-bit: one wave per
    # SIMD, 32-row streamed tiles in dK / dV; float32: one LDS stage), inputs
    # zero-padded.
    B, S, H = 2, 200, 3
    shape = (B, S, H, D) if layout == "BSHD" else (B, H, S, D)
    q, k, v, dout = (rnd(shape, 70 + i, dtype) for i in range(4))
    scale = 1 / math.sqrt(D)
    got = run_grads(lambda a, b, c: flash_attention(a, b, c, causal=causal, layout=layout),
                    device, q, k, v, dout)[1:]
    check_grads(got, q, k, v, dout, dtype, scale, causal, layout=layout)


@pytest.mark.parametrize("W,H,H_kv", [(33, 4, 4), (-1, 8, 2)])
def test_head_dim_256_grad_window_gqa(device, W, H, H_kv):
    # D = 256 gradients under a sliding window (W = 33) and with grouped K/V
    # heads (8 query heads over 2).
    dtype, B, Sq, Sk, D = torch.bfloat16, 2, 300, 300, 256
    q = rnd((B, Sq, H, D), 80, dtype)
    k, v = rnd((B, Sk, H_kv, D), 81, dtype), rnd((B, Sk, H_kv, D), 82, dtype)
    dout = rnd((B, Sq, H, D), 83, dtype)
    if W >= 0:
        fn = lambda a, b, c: sliding_window_attention(a, b, c, W)
    else:
        fn = lambda a, b, c: flash_attention(a, b, c, causal=True, enable_gqa=True)
    got = run_grads(fn, device, q, k, v, dout)[1:]
    check_grads(got, q, k, v, dout, dtype, 1 / math.sqrt(D), True, W)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("Sq,Sk,causal", [(77, 300, False), (300, 77, False), (77, 300, True),
                                          (300, 77, True), (1, 129, False), (129, 1, True)])
def test_flash_grad_ragged(device, dtype, Sq, Sk, causal):
    q = rnd((2, Sq, 4, 128), 1, dtype)
    k, v = rnd((2, Sk, 4, 128), 2, dtype), rnd((2, Sk, 4, 128), 3, dtype)
    d = rnd((2, Sq, 4, 128), 4, dtype)
    fn = lambda q, k, v: flash_attention(q, k, v, causal=causal)
    out, *g = run_grads(fn, device, q, k, v, d)
    if causal and Sk > Sq:  # SDPA's causal rule: bottom-right diagonal, j <= i + Sk - Sq
        check_grads(g, q, k, v, d, dtype, 1 / math.sqrt(128), False, -1, Sk - Sq)
    else:
        check_grads(g, q, k, v, d, dtype, 1 / math.sqrt(128), causal)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("W,causal", [(7, True), (16, False), (75, True), (0, True)])
def test_sliding_window_grad(device, dtype, W, causal):
    q, k, v, d = (rnd((2, 260, 3, 64), 10 + i, dtype) for i in range(4))
    fn = lambda q, k, v: sliding_window_attention(q, k, v, window_size=W, causal=causal)
    out, *g = run_grads(fn, device, q, k, v, d)
    check_grads(g, q, k, v, d, dtype, 1 / 8, causal, W, -1 if causal else W)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("H,H_kv,D", [(8, 2, 128), (6, 3, 64), (4, 1, 64)])
def test_gqa_grad(device, dtype, H, H_kv, D):
    q, d = rnd((2, 200, H, D), 20, dtype), rnd((2, 200, H, D), 21, dtype)
    k, v = rnd((2, 200, H_kv, D), 22, dtype), rnd((2, 200, H_kv, D), 23, dtype)
    fn = lambda q, k, v: flash_attention(q, k, v, causal=True, enable_gqa=True)
    out, *g = run_grads(fn, device, q, k, v, d)
    check_grads(g, q, k, v, d, dtype, 1 / math.sqrt(D), True)


# Both backward schedules at D = 128 (the recomputing one, which autograd takes
# by default, and the stored-dS one): masks, ragged and tiny sizes, a partial
# last key block, windows on one and both sides, grouped heads.
SCHEDULE_CASES = [  # (Sq, Sk, H, H_kv, causal, W): W = sliding window, None = flash
    (300, 300, 4, 4, True, None), (1000, 1000, 2, 2, True, None),
    (77, 300, 4, 4, False, None), (300, 77, 4, 4, True, None), (300, 77, 4, 4, False, None),
    (129, 1, 2, 2, True, None), (1, 129, 2, 2, False, None), (260, 260, 4, 4, True, 75),
    (260, 260, 4, 4, False, 40), (700, 700, 2, 2, True, 300), (500, 500, 8, 2, True, None),
]


@pytest.mark.parametrize("stored", [True, False])
@pytest.mark.parametrize("case", SCHEDULE_CASES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_backward_schedules_d128(device, monkeypatch, dtype, case, stored):
    Sq, Sk, H, H_kv, causal, W = case
    monkeypatch.setattr(_launch, "BWD_STORED_DS", stored)
    seed = Sq * 7 + Sk + H_kv
    q, d = rnd((2, Sq, H, 128), seed, dtype), rnd((2, Sq, H, 128), seed + 1, dtype)
    k, v = rnd((2, Sk, H_kv, 128), seed + 2, dtype), rnd((2, Sk, H_kv, 128), seed + 3, dtype)
    if W is None:
        fn = lambda q, k, v: flash_attention(q, k, v, causal=causal, enable_gqa=H != H_kv)
    else:
        fn = lambda q, k, v: sliding_window_attention(q, k, v, window_size=W, causal=causal)
    out, *g = run_grads(fn, device, q, k, v, d)
    if W is not None:
        check_grads(g, q, k, v, d, dtype, 1 / math.sqrt(128), causal, W, -1 if causal else W)
    elif causal and Sk > Sq:
        check_grads(g, q, k, v, d, dtype, 1 / math.sqrt(128), False, -1, Sk - Sq)
    else:
        check_grads(g, q, k, v, d, dtype, 1 / math.sqrt(128), causal)


def test_backward_schedules_agree(device, monkeypatch):
    # The two schedules differ only in summation order and in which kernel forms
    # Dvec: their gradients agree to a few bf16 rounding units, normwise.
    q, k, v, d = (rnd((2, 2048, 4, 128), 90 + i, torch.bfloat16) for i in range(4))
    fn = lambda q, k, v: flash_attention(q, k, v, causal=True)
    got = {}
    for stored in (True, False):
        monkeypatch.setattr(_launch, "BWD_STORED_DS", stored)
        got[stored] = run_grads(fn, device, q, k, v, d)[1:]
    for name, a, b in zip(("dq", "dk", "dv"), got[True], got[False]):
        a, b = a.double(), b.double()
        assert torch.isfinite(a).all(), name
        rel = float((a - b).norm() / b.norm())
        print(f"{name}: stored vs recompute normwise {rel:.2e}")
        assert rel <= 4e-3, name


@pytest.mark.parametrize("dtype", DTYPES)
def test_reference_gradient_flows(device, dtype):
    # tests/attention/test_flash.py:338-362 (loss = sum(out ** 2), causal; float32 there)
    q, k, v = (rnd((2, 32, 4, 64), s, dtype) for s in (42, 43, 44))
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    out = flash_attention(qd, kd, vd, causal=True)
    (out.float() ** 2).sum().backward()
    torch.cuda.synchronize()
    for x in (qd, kd, vd):
        assert x.grad.shape == x.shape and bool((x.grad != 0).any())
    d = (2 * out.detach().float()).to(dtype).cpu()
    check_grads((qd.grad, kd.grad, vd.grad), q, k, v, d, dtype, 1 / 8, True)


def test_reference_chunked_gradient_flows(device):
    # tests/attention/test_chunked.py:318-339 (q 16 tokens, k/v 64, chunk 16), in float16
    q = rnd((2, 16, 4, 32), 45, torch.float16)
    k, v = rnd((2, 64, 4, 32), 46, torch.float16), rnd((2, 64, 4, 32), 47, torch.float16)
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    out = chunked_cross_attention(qd, kd, vd, chunk_size=16)
    (out.float() ** 2).sum().backward()
    torch.cuda.synchronize()
    d = (2 * out.detach().float()).to(torch.float16).cpu()  # d(sum o^2)/do
    for x in (qd, kd, vd):
        assert bool((x.grad != 0).any())
    check_grads((qd.grad, kd.grad, vd.grad), q, k, v, d, torch.float16, 1 / math.sqrt(32), False)


@pytest.mark.parametrize("size", [(1, 64, 4, 32), (2, 256, 8, 64), (4, 1024, 16, 64)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_reference_parity_sizes_sum_loss(device, size, dtype):
    # tests/parity/pytorch/test_attention_parity.py:107-163: loss = sum(out), non-causal,
    # SIZE_CONFIGS tiny / small / medium (tests/parity/shared/input_generators.py:12-44)
    q, k, v = (rnd(size, 42 + i, dtype) for i in range(3))
    qd, kd, vd = (x.to(device).requires_grad_(True) for x in (q, k, v))
    flash_attention(qd, kd, vd, causal=False).sum().backward()
    torch.cuda.synchronize()
    ones = torch.ones(size, dtype=dtype)
    check_grads((qd.grad, kd.grad, vd.grad), q, k, v, ones, dtype, 1 / math.sqrt(size[-1]),
                False)


def test_deterministic(device):
    q, k, v, d = (rnd((2, 700, 4, 128), 50 + i, torch.bfloat16) for i in range(4))
    fn = lambda q, k, v: flash_attention(q, k, v, causal=True)
    a = run_grads(fn, device, q, k, v, d)
    b = run_grads(fn, device, q, k, v, d)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_headline_shape_sampled_heads(device):
    # (4, 32, 4096, 128) bf16 causal BHSD: full-size backward, two (batch, head)
    # slices checked against the oracle, all gradients finite.
    B, H, S, D = 4, 32, 4096, 128
    q, k, v, d = (rnd((B, H, S, D), 60 + i, torch.bfloat16) for i in range(4))
    fn = lambda q, k, v: flash_attention(q, k, v, causal=True, layout="BHSD")
    out, dq, dk, dv = run_grads(fn, device, q, k, v, d)
    for x in (dq, dk, dv):
        assert bool(torch.isfinite(x).all())
    for b, h in ((0, 0), (3, 31)):
        sl = lambda x: x[b:b + 1, h:h + 1]
        check_grads((sl(dq), sl(dk), sl(dv)), sl(q), sl(k), sl(v), sl(d), torch.bfloat16,
                    1 / math.sqrt(D), True, layout="BHSD")


@pytest.mark.parametrize("stored", [False, True])
def test_paired_tiles_single_tail(device, monkeypatch, stored):
    # 136 (batch, head)s over the 8 XCDs (17 each) with 8 tiles of 128 rows.
    # Stored dS: each XCD runs the dK/dV tile pairs of its first head, then the
    # tiles of the other 16 one per workgroup; XCD x holds heads x, x + 8, ...,
    # so the sample takes both kinds on several XCDs. Recomputing: pairs only.
    monkeypatch.setattr(_launch, "BWD_STORED_DS", stored)
    B, H, S, D = 1, 136, 1024, 128
    q, k, v, d = (rnd((B, H, S, D), 70 + i, torch.bfloat16) for i in range(4))
    fn = lambda q, k, v: flash_attention(q, k, v, causal=True, layout="BHSD")
    out, dq, dk, dv = run_grads(fn, device, q, k, v, d)
    for x in (dq, dk, dv):
        assert bool(torch.isfinite(x).all())
    for h in (0, 3, 8, 13, 64, 101, 128, 135):
        sl = lambda x: x[:, h:h + 1]
        check_grads((sl(dq), sl(dk), sl(dv)), sl(q), sl(k), sl(v), sl(d), torch.bfloat16,
                    1 / math.sqrt(D), True, layout="BHSD")


def test_forward_matches_no_grad_path(device):
    # the differentiable forward (row log-sum-exp kept) returns the same output
    q, k, v = (rnd((2, 333, 4, 128), 70 + i, torch.bfloat16).to(device) for i in range(3))
    with torch.no_grad():
        ref = flash_attention(q, k, v, causal=True)
    qg = q.clone().requires_grad_(True)
    out = flash_attention(qg, k, v, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(out.detach(), ref)


def test_unsupported_grad_cases_raise(device):
    y = torch.randn(1, 16, 2, 64, device=device, dtype=torch.bfloat16, requires_grad=True)
    with pytest.raises(NotImplementedError, match="scale > 0"):
        flash_attention(y, y, y, scale=-0.1, causal=True)
    with torch.no_grad():
        flash_attention(y, y, y, scale=-0.1, causal=True)  # the forward still runs


def test_float32_headline_shape_sampled_heads(device):
    # float32 at a large shape: (2, 8, 2048, 128) causal BSHD, two (batch, head)
    # slices against the oracle.
    B, S, H, D = 2, 2048, 8, 128
    q, k, v, d = (rnd((B, S, H, D), 80 + i, torch.float32) for i in range(4))
    fn = lambda q, k, v: flash_attention(q, k, v, causal=True)
    out, dq, dk, dv = run_grads(fn, device, q, k, v, d)
    for b, h in ((0, 0), (1, 7)):
        sl = lambda x: x[b:b + 1, :, h:h + 1]
        check_grads((sl(dq), sl(dk), sl(dv)), sl(q), sl(k), sl(v), sl(d), torch.float32,
                    1 / math.sqrt(D), True)

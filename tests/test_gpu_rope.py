"""GPU parity of RoPE and fused RoPE + flash attention (HIP kernels through the
C ABI) against the CPU oracle (oracle/rope.py).

Tolerances: float32 rtol 1e-4 / atol 1e-5 (rope alone: 1e-5); float16 /
bfloat16 max-abs <= 2e-2 against the float64 oracle on the same cast inputs.
The reference rotates in the input dtype (kernels/rope.py:477-497), so the
16-bit oracle attention runs on rotated Q/K rounded to that dtype.
"""

import math

import numpy as np
import pytest
import torch

from mlx_primitives.attention import flash_attention
from mlx_primitives.kernels import (
    FusedRoPEFlashAttention,
    fast_fused_rope_attention,
    fused_rope_attention,
    precompute_rope_cache,
    rope,
)
from oracle import rope as orope

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def rnd(shape, seed, dtype, mult=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * mult).to(dtype)


def check(out, ref, dtype, rope_only=False):
    got = out.double().cpu().numpy()
    assert got.shape == ref.shape
    if dtype == torch.float32:
        tol = 1e-5 if rope_only else 1e-4
        np.testing.assert_allclose(got, ref, rtol=tol, atol=1e-5)
    else:
        err = float(np.abs(got - ref).max())
        assert err <= 2e-2, f"max abs err {err}"


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("cache_dt", ["f32", "same"])
def test_rope_kernel(device, dt, D, cache_dt):
    dtype = DT[dt]
    x = rnd((2, 37, 3, D), D, dtype)
    cdt = torch.float32 if cache_dt == "f32" else dtype
    cos, sin = precompute_rope_cache(60, D, dtype=cdt, device=device)
    out = rope(x.to(device), cos, sin, offset=11)
    ref = orope.rope(x.double().numpy(), cos.double().cpu().numpy(), sin.double().cpu().numpy(), 11)
    check(out, ref, dtype, rope_only=True)


def test_rope_strided_input_and_out(device):
    # a (B, S, H, D) view of a head-major tensor, written into a given buffer
    xh = rnd((2, 4, 50, 64), 3, torch.bfloat16).to(device)
    x = xh.transpose(1, 2)
    assert not x.is_contiguous()
    cos, sin = precompute_rope_cache(50, 64, dtype=torch.bfloat16, device=device)
    out = torch.empty(2, 50, 4, 64, dtype=torch.bfloat16, device=device)
    res = rope(x, cos, sin, 0, out=out)
    assert res.data_ptr() == out.data_ptr()
    ref = orope.rope(x.double().cpu().numpy(), cos.double().cpu().numpy(),
                     sin.double().cpu().numpy(), 0)
    check(out, ref, torch.bfloat16, rope_only=True)


def test_rope_position_zero_is_identity(device):
    x = rnd((1, 1, 8, 128), 4, torch.float32).to(device)
    cos, sin = precompute_rope_cache(4, 128, device=device)
    assert torch.equal(rope(x, cos, sin, 0), x)


def oracle_attention(q, k, v, dtype, scale, q_off, kv_off, causal, base=10000.0):
    """Float64 oracle with Q/K rotated on the reference's cache and rounded to dtype."""
    D = q.shape[-1]
    n = max(q.shape[1] + q_off, k.shape[1] + kv_off)
    cos, sin = precompute_rope_cache(n, D, base=base, dtype=dtype)
    c64, s64 = cos.double().numpy(), sin.double().numpy()
    qr = torch.from_numpy(orope.rope(q.double().numpy(), c64, s64, q_off)).to(dtype)
    kr = torch.from_numpy(orope.rope(k.double().numpy(), c64, s64, kv_off)).to(dtype)
    one, zero = np.ones((n, D // 2)), np.zeros((n, D // 2))
    return orope.fused_rope_attention(qr.double().numpy(), kr.double().numpy(),
                                      v.double().numpy(), scale, one, zero, q_offset=q_off,
                                      kv_offset=kv_off, causal=causal)


# tests/correctness/test_fused_rope_attention_correctness.py:79-295 (shapes,
# offsets, bases)
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("qs,ks,q_off,kv_off,causal", [
    ((1, 64, 4, 64), (1, 64, 4, 64), 0, 0, True),
    ((1, 64, 4, 64), (1, 64, 4, 64), 0, 0, False),
    ((1, 1, 4, 64), (1, 32, 4, 64), 31, 0, True),     # decode, 139-160
    ((1, 8, 4, 64), (1, 8, 4, 64), 16, 16, True),     # both offsets, 162-183
    ((2, 1, 4, 64), (2, 64, 4, 64), 63, 0, True),     # q shorter, 189-209
    ((2, 32, 4, 64), (2, 16, 4, 64), 0, 0, False),    # q longer, 211-232
    ((2, 40, 3, 128), (2, 72, 3, 128), 50, 10, True),
    # kv_offset > q_offset: the first 15 queries precede every key (zeros)
    ((2, 40, 3, 64), (2, 48, 3, 64), 5, 20, True),
    ((1, 300, 2, 128), (1, 260, 2, 128), 0, 37, True),
    ((1, 16, 2, 64), (1, 16, 2, 64), 0, 100, True),    # no query sees a key
])
def test_fused_rope_attention(device, dt, qs, ks, q_off, kv_off, causal):
    dtype = DT[dt]
    q, k, v = rnd(qs, 1, dtype), rnd(ks, 2, dtype), rnd(ks, 3, dtype)
    scale = 1 / math.sqrt(qs[-1])
    out = fused_rope_attention(q.to(device), k.to(device), v.to(device), q_offset=q_off,
                               kv_offset=kv_off, causal=causal)
    assert out.shape == qs and out.dtype == dtype
    check(out, oracle_attention(q, k, v, dtype, scale, q_off, kv_off, causal), dtype)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("qs,ks,q_off,kv_off", [
    ((1, 4, 4, 64), (1, 64, 4, 64), 0, 0),      # zero offsets, Sq < Skv: bottom right
    ((2, 1, 4, 64), (2, 64, 4, 64), 63, 0),     # decode step
    ((1, 8, 4, 64), (1, 8, 4, 64), 16, 16),
    ((2, 40, 3, 128), (2, 24, 3, 128), 3, 10),  # Sq > Skv: top left; kv_offset > q_offset
])
def test_fast_fused_rope_attention_sdpa_rule(device, dt, qs, ks, q_off, kv_off):
    # fast_fused_rope_attention hands mask="causal" to SDPA
    # (fused_rope_attention.py:716-727): offsets rotate only.
    dtype = DT[dt]
    q, k, v = rnd(qs, 21, dtype), rnd(ks, 22, dtype), rnd(ks, 23, dtype)
    out = fast_fused_rope_attention(q.to(device), k.to(device), v.to(device), q_offset=q_off,
                                    kv_offset=kv_off, causal=True)
    D = qs[-1]
    n = max(qs[1] + q_off, ks[1] + kv_off)
    cos, sin = precompute_rope_cache(n, D, dtype=dtype)
    c64, s64 = cos.double().numpy(), sin.double().numpy()
    qr = torch.from_numpy(orope.rope(q.double().numpy(), c64, s64, q_off)).to(dtype)
    kr = torch.from_numpy(orope.rope(k.double().numpy(), c64, s64, kv_off)).to(dtype)
    one, zero = np.ones((n, D // 2)), np.zeros((n, D // 2))
    ref = orope.fast_fused_rope_attention(qr.double().numpy(), kr.double().numpy(),
                                          v.double().numpy(), 1 / math.sqrt(D), one, zero,
                                          q_offset=q_off, kv_offset=kv_off, causal=True)
    check(out, ref, dtype)


@pytest.mark.parametrize("base", [10000.0, 500000.0, 100.0])
def test_rope_bases(device, base):
    # test_fused_rope_attention_correctness.py:271-295
    q, k, v = (rnd((1, 48, 4, 64), s, torch.bfloat16) for s in (5, 6, 7))
    out = fast_fused_rope_attention(q.to(device), k.to(device), v.to(device), rope_base=base,
                                    causal=True)
    ref = oracle_attention(q, k, v, torch.bfloat16, 1 / 8, 0, 0, True, base=base)
    check(out, ref, torch.bfloat16)


@pytest.mark.parametrize("mult", [10.0, 1e-3])
def test_extreme_values_finite(device, mult):
    # test_fused_rope_attention_correctness.py:238-268
    q, k, v = (rnd((1, 64, 4, 64), s, torch.float16, mult) for s in (8, 9, 10))
    out = fused_rope_attention(q.to(device), k.to(device), v.to(device), causal=True)
    assert torch.isfinite(out.float()).all()


def test_given_caches_and_validation(device):
    q, k, v = (rnd((1, 16, 2, 64), s, torch.bfloat16).to(device) for s in (11, 12, 13))
    cos, sin = precompute_rope_cache(16, 64, dtype=torch.bfloat16, device=device)
    a = fused_rope_attention(q, k, v, cos_cache=cos, sin_cache=sin, causal=True)
    b = fused_rope_attention(q, k, v, causal=True)
    assert torch.equal(a, b)
    with pytest.raises(ValueError, match="4D"):
        fused_rope_attention(q[0], k, v)
    with pytest.raises(ValueError, match="exceed"):
        fused_rope_attention(q, k, v, cos_cache=cos[:8], sin_cache=sin[:8])
    # keys placed after the first queries: those rows are zeros, the rest is
    # the attention of the later rows (fused_rope_attention.py:127-131, 176-186)
    z = fused_rope_attention(q, k, v, q_offset=0, kv_offset=4, causal=True)
    assert torch.equal(z[:, :4], torch.zeros_like(z[:, :4]))
    assert torch.isfinite(z.float()).all() and z[:, 4:].abs().amax() > 0


def test_serving_shape_matches_flash_on_rotated_inputs(device):
    # Same kernels: fused RoPE attention == flash_attention on rope(Q), rope(K),
    # bit for bit, at a serving shape; rows sampled against the oracle.
    q, k, v = (rnd((2, 2048, 16, 128), s, torch.bfloat16).to(device) for s in (14, 15, 16))
    out = fused_rope_attention(q, k, v, causal=True)
    cos, sin = precompute_rope_cache(2048, 128, dtype=torch.bfloat16, device=device)
    ref = flash_attention(rope(q, cos, sin), rope(k, cos, sin), v, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_module_incremental_decoding(device):
    # Running the module over S+1 tokens at once equals running S tokens, then
    # one token with the returned cache at offset S (last row).
    torch.manual_seed(0)
    m = FusedRoPEFlashAttention(dims=256, num_heads=4, causal=True, device=device,
                                dtype=torch.float32)
    x = torch.randn(2, 33, 256, device=device)
    with pytest.raises(NotImplementedError, match="forward pass only"):
        m(x)  # parameters require grad and grad mode is on
    with torch.no_grad():
        full, _ = m(x)
        part, cache = m(x[:, :32])
        step, cache2 = m(x[:, 32:33], cache=cache, offset=32)
    assert full.shape == (2, 33, 256) and cache2[0].shape == (2, 33, 4, 64)
    torch.testing.assert_close(part, full[:, :32], rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(step[:, 0], full[:, 32], rtol=1e-4, atol=1e-5)


def test_module_matches_oracle(device):
    torch.manual_seed(1)
    m = FusedRoPEFlashAttention(dims=128, num_heads=2, causal=True, device=device,
                                dtype=torch.float32)
    x = torch.randn(1, 20, 128, device=device)
    with torch.no_grad():
        out, _ = m(x)
        xs = x.double().cpu()
        proj = lambda lin: (xs @ lin.weight.double().cpu().T).reshape(1, 20, 2, 64).numpy()
        att = orope.fused_rope_attention(proj(m.q_proj), proj(m.k_proj), proj(m.v_proj),
                                         causal=True)
        ref = torch.from_numpy(att).reshape(1, 20, 128) @ m.out_proj.weight.double().cpu().T
    np.testing.assert_allclose(out.double().cpu().numpy(), ref.numpy(), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("D", [32, 64, 128, 80])
@pytest.mark.parametrize("cache_dt", ["same", "f32"])
@pytest.mark.parametrize("q_off,kv_off,causal", [(0, 0, True), (37, 5, True), (9, 9, False)])
def test_q_rotation_on_load_bit_identical(device, dt, D, cache_dt, q_off, kv_off, causal):
    # 16-bit, D in (32, 64, 128): the flash kernel rotates Q as it loads it; the
    # result equals the RoPE kernel followed by the flash kernel bit for bit
    # (same rotation arithmetic and rounding). D = 80 takes the RoPE-kernel path.
    dtype = DT[dt]
    q = rnd((2, 70, 3, D), 21, dtype).to(device)
    k = rnd((2, 90, 3, D), 22, dtype).to(device)
    v = rnd((2, 90, 3, D), 23, dtype).to(device)
    cdt = torch.float32 if cache_dt == "f32" else dtype
    n = max(70 + q_off, 90 + kv_off) + 3
    cos, sin = precompute_rope_cache(n, D, dtype=cdt, device=device)
    out = fused_rope_attention(q, k, v, cos_cache=cos, sin_cache=sin, q_offset=q_off,
                               kv_offset=kv_off, causal=causal)
    qr, kr = rope(q, cos, sin, q_off), rope(k, cos, sin, kv_off)
    shift = q_off - kv_off
    if causal:
        # the position rule kv_offset + j <= q_offset + i (top-left when shift == 0;
        # flash_attention's causal rule would align Sq < Sk at the bottom right)
        from mlx_primitives.attention._launch import run_attention
        from mlx_primitives.constants import Layout
        ref = run_attention(qr, kr, v, Layout.BSHD, 1 / math.sqrt(D), shift == 0,
                            window_right=shift if shift else -1)
    else:
        ref = flash_attention(qr, kr, v, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)

"""Host-side behaviour of the drop-in API (no GPU): argument validation with the
reference's messages, the no-CPU-fallback rule, and the pure host helpers."""

import numpy as np
import pytest
import torch

from mlx_primitives.attention import (
    ChunkedCrossAttention,
    FlashAttention,
    SlidingWindowAttention,
    chunked_cross_attention,
    create_sliding_window_mask,
    estimate_memory_savings,
    flash_attention,
    get_optimal_flash_config,
    sliding_window_attention,
)
from mlx_primitives.cache import (
    create_block_table_from_lengths,
    get_alibi_slopes,
    paged_attention,
    paged_attention_with_bias,
    set_block_data,
    store_kv,
)
from mlx_primitives.constants import Layout
from oracle import paged as op


def t(*shape, dtype=torch.float32):
    return torch.zeros(shape, dtype=dtype)


def test_flash_validation_messages():
    with pytest.raises(ValueError, match="Expected 4D tensors, got 3D"):
        flash_attention(t(1, 2, 3), t(1, 2, 3, 4), t(1, 2, 3, 4))
    with pytest.raises(ValueError, match="Expected K to be 4D"):
        flash_attention(t(1, 2, 3, 4), t(2, 3, 4), t(1, 2, 3, 4))
    with pytest.raises(ValueError, match="layout must be"):
        flash_attention(t(1, 2, 3, 4), t(1, 2, 3, 4), t(1, 2, 3, 4), layout="SBHD")
    with pytest.raises(ValueError, match="Batch size mismatch"):
        flash_attention(t(1, 2, 3, 4), t(2, 2, 3, 4), t(1, 2, 3, 4))
    with pytest.raises(ValueError, match="Number of heads mismatch"):
        flash_attention(t(1, 2, 3, 4), t(1, 2, 5, 4), t(1, 2, 5, 4))
    with pytest.raises(ValueError, match="Head dimension mismatch between Q and K"):
        flash_attention(t(1, 2, 3, 4), t(1, 2, 3, 8), t(1, 2, 3, 4))
    with pytest.raises(ValueError, match="Sequence length mismatch between K and V"):
        flash_attention(t(1, 2, 3, 4), t(1, 5, 3, 4), t(1, 6, 3, 4))
    with pytest.raises(ValueError, match="dtype mismatch"):
        flash_attention(t(1, 2, 3, 4), t(1, 2, 3, 4, dtype=torch.float16), t(1, 2, 3, 4))
    # BHSD reads heads from dim 1
    with pytest.raises(ValueError, match="Number of heads mismatch"):
        flash_attention(t(1, 2, 3, 4), t(1, 3, 3, 4), t(1, 3, 3, 4), layout=Layout.BHSD)


def test_no_cpu_fallback():
    x = t(1, 8, 2, 64)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        flash_attention(x, x, x)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        sliding_window_attention(x, x, x, window_size=2)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        chunked_cross_attention(x, x, x)
    q = t(2, 1, 2, 64); pool = t(4, 16, 2, 64)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        paged_attention(q, pool, pool, torch.zeros(2, 1, dtype=torch.int32),
                        torch.ones(2, dtype=torch.int32))


def test_dropout_validated_and_no_cpu_fallback():
    x = t(1, 8, 2, 64)
    with pytest.raises(ValueError, match="dropout_p"):
        flash_attention(x, x, x, dropout_p=1.0)
    with pytest.raises(ValueError, match="dropout_p"):
        sliding_window_attention(x, x, x, 2, dropout_p=1.0)
    with pytest.raises(ValueError, match="dropout_p"):
        chunked_cross_attention(x, x, x, dropout_p=2.0)
    # a valid rate runs on the GPU kernels only
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        flash_attention(x, x, x, dropout_p=0.1)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        sliding_window_attention(x, x, x, 2, dropout_p=0.1)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        chunked_cross_attention(x, x, x, dropout_p=0.1)


def test_paged_validation():
    q = t(2, 1, 2, 64); pool = t(4, 16, 2, 64)
    tables = torch.zeros(2, 1, dtype=torch.int32); lens = torch.ones(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="block_size"):
        paged_attention(q, pool, pool, tables, lens, block_size=8)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        paged_attention(t(2, 3, 2, 64), pool, pool, tables, lens)  # prefill: no CPU path
    with pytest.raises(ValueError, match="Cannot specify both"):
        paged_attention_with_bias(q, pool, pool, tables, lens, attention_bias=q,
                                  alibi_slopes=torch.ones(2))
    with pytest.raises(NotImplementedError):
        paged_attention_with_bias(q, pool, pool, tables, lens, attention_bias=q)


def test_module_defaults():
    assert FlashAttention(8, 64).block_q == 32 and FlashAttention(8, 128).block_kv == 16
    assert FlashAttention(8, 128, block_q=8, block_kv=8).block_q == 8
    assert SlidingWindowAttention(8, 64, 32).scale == pytest.approx(0.125)
    assert ChunkedCrossAttention(8, 64).chunk_size == 1024


def test_optimal_config_kats():
    # tests/attention/test_flash.py:315-336
    bq, bk = get_optimal_flash_config(1024, 32, 8)
    assert bq >= 16 and bk >= 16
    bq, bk = get_optimal_flash_config(1024, 128, 8)
    assert bq <= 32 and bk <= 32
    bq, bk = get_optimal_flash_config(16, 64, 8)
    assert bq <= 16 and bk <= 16


def test_memory_savings():
    dense, chunk, ratio = estimate_memory_savings(512, 65536, 16, 64, 1024)
    assert dense == 512 * 65536 * 16 * 4 and chunk == 512 * 1024 * 16 * 4 and ratio == 64


def test_sliding_window_mask_kats():
    # tests/attention/test_sliding_window.py:74-103
    causal = create_sliding_window_mask(5, 2, causal=True).int().tolist()
    assert causal == [[1, 0, 0, 0, 0], [1, 1, 0, 0, 0], [1, 1, 1, 0, 0], [0, 1, 1, 1, 0],
                      [0, 0, 1, 1, 1]]
    bi = create_sliding_window_mask(5, 1, causal=False).int().tolist()
    assert bi == [[1, 1, 0, 0, 0], [1, 1, 1, 0, 0], [0, 1, 1, 1, 0], [0, 0, 1, 1, 1],
                  [0, 0, 0, 1, 1]]


@pytest.mark.parametrize("lens,bs", [([16, 32, 48], 16), ([10, 25], 16), ([1, 100, 7], 8)])
def test_block_tables_match_oracle(lens, bs):
    got = create_block_table_from_lengths(torch.tensor(lens, dtype=torch.int32), bs)
    np.testing.assert_array_equal(got.numpy(), op.create_block_table_from_lengths(np.array(lens), bs))
    assert got.dtype == torch.int32


def test_alibi_slopes_match_oracle():
    for h in (1, 8, 12, 32):
        np.testing.assert_allclose(get_alibi_slopes(h).numpy(), op.get_alibi_slopes(h), rtol=1e-7)


def test_store_kv_validation():
    pool = t(8, 16, 2, 64); x = t(2, 3, 2, 64); tables = torch.zeros(2, 1, dtype=torch.int32)
    with pytest.raises(ValueError, match="k and v"):
        store_kv(pool, pool, tables, x, t(2, 3, 2, 32), 0)
    with pytest.raises(ValueError, match="heads/dim"):
        store_kv(pool, pool, tables, t(2, 3, 4, 64), t(2, 3, 4, 64), 0)
    with pytest.raises(ValueError, match="dtype"):
        store_kv(pool, pool, tables, x.half(), x.half(), 0)
    with pytest.raises(ValueError, match="block_tables"):
        store_kv(pool, pool, tables[:1], x, x, 0)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        store_kv(pool, pool, tables, x, x, 0)
    with pytest.raises(ValueError, match="block_id"):
        set_block_data(pool, pool, 8, x[0], x[0])
    with pytest.raises(ValueError, match="fit"):
        set_block_data(pool, pool, 0, t(4, 2, 64), t(4, 2, 64), start_pos=14)


def test_rope_host_validation():
    from mlx_primitives.kernels import fused_rope_attention, precompute_rope_cache, rope
    from oracle import rope as orope

    x = t(1, 4, 2, 64)
    cos, sin = precompute_rope_cache(4, 64)
    c64, s64 = orope.precompute_rope_cache(4, 64)
    # same float32 formula (torch's and numpy's float32 cos/sin differ by an ulp)
    np.testing.assert_allclose(cos.numpy(), c64, rtol=0, atol=1e-6)
    np.testing.assert_allclose(sin.numpy(), s64, rtol=0, atol=1e-6)
    with pytest.raises(ValueError, match="even"):
        precompute_rope_cache(4, 7)
    with pytest.raises(ValueError, match="exceed"):
        rope(x, cos, sin, offset=1)
    with pytest.raises(NotImplementedError, match="multiple of 16"):
        rope(t(1, 4, 2, 40), *precompute_rope_cache(4, 40))
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        rope(x, cos, sin)
    with pytest.raises(ValueError, match="Q must be 4D"):
        fused_rope_attention(x[0], x, x)
    with pytest.raises(ValueError, match="even"):
        fused_rope_attention(t(1, 4, 2, 63), t(1, 4, 2, 63), t(1, 4, 2, 63))


def test_forward_only_guard():
    from mlx_primitives import _native

    x = t(1, 4, 2, 64).requires_grad_()
    with pytest.raises(NotImplementedError, match="forward pass only"):
        _native.require_no_grad(x)
    with torch.no_grad():
        _native.require_no_grad(x)
    _native.require_no_grad(x.detach(), None)


def test_gqa_flag_validation():
    q, k = t(1, 8, 6, 64), t(1, 8, 2, 64)
    with pytest.raises(ValueError, match="Number of heads mismatch"):
        flash_attention(q, k, k)
    with pytest.raises(ValueError, match="enable_gqa"):
        flash_attention(q, t(1, 8, 4, 64), t(1, 8, 4, 64), enable_gqa=True)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        flash_attention(q, k, k, enable_gqa=True)  # validation passes, no CPU path
    qd = t(2, 1, 8, 64); pool = t(4, 16, 2, 64)
    tables = torch.zeros(2, 1, dtype=torch.int32); lens = torch.ones(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="pool heads"):
        paged_attention(qd, pool, pool, tables, lens)
    with pytest.raises(ValueError, match="divide"):
        paged_attention(qd, t(4, 16, 3, 64), t(4, 16, 3, 64), tables, lens, enable_gqa=True)
    with pytest.raises(RuntimeError, match="ROCm device tensors only"):
        paged_attention(qd, pool, pool, tables, lens, enable_gqa=True)

"""C-ABI checks that need no GPU: the library loads, exports every function
declared in include/mpx_attn.h, and rejects bad arguments before any HIP call."""

import ctypes
import os
import re

import numpy as np
import pytest
import torch  # noqa: F401  (loads the HIP runtime the library links against)

from mlx_primitives import _native

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "include", "mpx_attn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mpx_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_native.library_path()):
        pytest.skip("libmpx_attn.so not built")
    return _native.load()


def test_header_declares_expected_entry_points():
    assert declared_functions() == sorted([
        "mpx_version", "mpx_last_error", "mpx_attn_fwd", "mpx_attn_fwd_workspace_bytes",
        "mpx_paged_decode", "mpx_paged_decode_workspace_bytes", "mpx_paged_prefill",
        "mpx_paged_prefill_workspace_bytes", "mpx_kv_append", "mpx_rope", "mpx_attn_fwd_gqa",
        "mpx_paged_decode_gqa", "mpx_paged_prefill_gqa", "mpx_attn_fwd_lse", "mpx_attn_bwd",
        "mpx_attn_bwd_workspace_bytes", "mpx_attn_fwd_rope", "mpx_paged_decode_noalloc",
        "mpx_rope_at", "mpx_kv_append_rope", "mpx_attn_fwd_dropout", "mpx_attn_bwd_dropout",
        "mpx_attn_bwd_ds_workspace_bytes"])


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert ctypes.cast(getattr(lib, name), ctypes.c_void_p).value


def test_version(lib):
    assert lib.mpx_version() == (0 << 16) | 1


def _fwd(lib, dtype=2, D=64, B=1, H=1, Sq=8, Sk=8, scale=0.1, ptr=16):
    st = (ctypes.c_int64 * 3)(8 * 64, 8 * 64, 64)
    return lib.mpx_attn_fwd(ptr, ptr, ptr, ptr, st, st, st, st, B, H, Sq, Sk, D, scale, 1, -1,
                            -1, dtype, None, 0, None)


def test_fwd_rejects_bad_dtype(lib):
    assert _fwd(lib, dtype=7) == _native.MPX_EINVAL
    assert b"dtype" in lib.mpx_last_error()


def test_fwd_unsupported_head_dim(lib):
    assert _fwd(lib, D=96) == _native.MPX_EUNSUPPORTED
    assert b"head_dim" in lib.mpx_last_error()


def test_fwd_rejects_misaligned_pointer(lib):
    assert _fwd(lib, ptr=18) == _native.MPX_EINVAL
    assert b"aligned" in lib.mpx_last_error()


def test_fwd_rejects_nonfinite_scale(lib):
    assert _fwd(lib, scale=float("nan")) == _native.MPX_EINVAL


def test_fwd_empty_problem_is_noop(lib):
    assert _fwd(lib, B=0) == _native.MPX_OK
    assert lib.mpx_last_error() == b""


def test_fwd_workspace_sizes(lib):
    # Few q-tiles and a long KV range -> split-KV partials are needed.
    ws = lib.mpx_attn_fwd_workspace_bytes(1, 16, 512, 65536, 64, 0, -1, -1, 2)
    assert ws > 0 and ws % (4 * (64 + 2)) == 0
    # config 1 (fp32 causal 2 x 12 heads x 1024, D = 64): q-tiles of 128 rows split
    # 1, 1, 2, 2, 3, 3, 4, 4 ways (pieces of 4 tiles of 64 keys): 4 partial slots
    assert lib.mpx_attn_fwd_workspace_bytes(2, 12, 1024, 1024, 64, 1, -1, -1, 0) == \
        4 * 2 * 12 * 1024 * (64 + 2) * 4
    # Enough q-tiles to fill the GPU -> no workspace.
    assert lib.mpx_attn_fwd_workspace_bytes(4, 32, 4096, 4096, 128, 1, -1, -1, 2) == 0


def test_paged_workspace_and_validation(lib):
    need = lib.mpx_paged_decode_workspace_bytes(64, 32, 128, 16, 512)
    assert need == 64 * 32 * 16 * (128 + 2) * 4
    st = (ctypes.c_int64 * 2)(4096, 128)
    rc = lib.mpx_paged_decode(16, 16, 16, 16, 16, None, 16, st, st, 1, 32, 128, 4, 0, 1, 0.1, 1,
                              16, 1 << 20, None)
    assert rc == _native.MPX_EINVAL and b"block_size" in lib.mpx_last_error()
    rc = lib.mpx_paged_decode(16, 16, 16, 16, 16, None, 16, st, st, 1, 32, 128, 4, 16, 1, 0.1, 1,
                              16, 8, None)
    assert rc == _native.MPX_EINVAL and b"workspace" in lib.mpx_last_error()


def _prefill(lib, dtype=1, D=128, bs=16, ws=None, ws_bytes=0, B=1, Sq=64, scale=0.1):
    st = (ctypes.c_int64 * 3)(64 * 32 * 128, 128, 32 * 128)
    return lib.mpx_paged_prefill(16, 16, 16, 16, 16, None, 16, st, st, B, Sq, 32, D, 64, bs, 8,
                                 scale, 1, dtype, ws, ws_bytes, None)


def test_paged_prefill_validation(lib):
    assert _prefill(lib, dtype=5) == _native.MPX_EINVAL and b"dtype" in lib.mpx_last_error()
    assert _prefill(lib, D=96) == _native.MPX_EUNSUPPORTED
    assert b"head_dim" in lib.mpx_last_error()
    assert _prefill(lib, bs=0) == _native.MPX_EINVAL and b"block_size" in lib.mpx_last_error()
    assert _prefill(lib, scale=float("inf")) == _native.MPX_EINVAL
    assert _prefill(lib, B=0) == _native.MPX_OK and lib.mpx_last_error() == b""
    # one sequence, 64 queries over 8 pages of 16: no split, no workspace
    assert lib.mpx_paged_prefill_workspace_bytes(1, 64, 32, 128, 16, 8, 1, 1) == 0
    # few queries over a long table: split-KV partials are needed
    need = lib.mpx_paged_prefill_workspace_bytes(1, 64, 8, 128, 16, 4096, 0, 1)
    assert need > 0
    st = (ctypes.c_int64 * 3)(64 * 8 * 128, 128, 8 * 128)
    rc = lib.mpx_paged_prefill(16, 16, 16, 16, 16, None, 16, st, st, 1, 64, 8, 128, 4096, 16,
                               4096, 0.1, 0, 1, 16, need - 1, None)
    assert rc == _native.MPX_EINVAL and b"workspace" in lib.mpx_last_error()


def _append(lib, dtype=2, D=128, B=2, T=4, bs=16, errors=16):
    st = (ctypes.c_int64 * 3)(T * 8 * D, 8 * D, D)
    return lib.mpx_kv_append(16, 16, 16, 16, 16, 16, 16, st, st, B, T, 8, D, 32, bs, 4, dtype,
                             errors, None)


def test_kv_append_validation(lib):
    assert _append(lib, dtype=9) == _native.MPX_EINVAL and b"dtype" in lib.mpx_last_error()
    assert _append(lib, D=4) == _native.MPX_EINVAL and b"16 bytes" in lib.mpx_last_error()
    assert _append(lib, bs=0) == _native.MPX_EINVAL
    assert _append(lib, errors=None) == _native.MPX_EINVAL and b"null" in lib.mpx_last_error()
    assert _append(lib, B=0) == _native.MPX_OK and lib.mpx_last_error() == b""


def _rope(lib, dtype=2, cdt=2, D=128, S=8, offset=0, n_pos=8, ptr=16):
    st = (ctypes.c_int64 * 3)(S * 4 * D, 4 * D, D)
    return lib.mpx_rope(ptr, ptr, ptr, ptr, st, st, 1, S, 4, D, offset, n_pos, dtype, cdt, None)


def test_rope_validation(lib):
    assert _rope(lib, dtype=4) == _native.MPX_EINVAL and b"dtype" in lib.mpx_last_error()
    assert _rope(lib, cdt=-1) == _native.MPX_EINVAL and b"cache" in lib.mpx_last_error()
    assert _rope(lib, D=72) == _native.MPX_EINVAL and b"multiple of 16" in lib.mpx_last_error()
    assert _rope(lib, offset=3) == _native.MPX_EINVAL and b"exceed" in lib.mpx_last_error()
    assert _rope(lib, ptr=24) == _native.MPX_EINVAL and b"aligned" in lib.mpx_last_error()
    assert _rope(lib, S=0) == _native.MPX_OK and lib.mpx_last_error() == b""


def test_rope_at_and_append_rope_validation(lib):
    st = (ctypes.c_int64 * 3)(8 * 4 * 128, 4 * 128, 128)
    rc = lib.mpx_rope_at(16, 16, 16, 16, st, st, 1, 8, 4, 72, 16, 8, 2, 2, 16, None)
    assert rc == _native.MPX_EINVAL and b"multiple of 16" in lib.mpx_last_error()
    rc = lib.mpx_rope_at(16, 16, 16, 16, st, st, 1, 8, 4, 128, None, 8, 2, 2, 16, None)
    assert rc == _native.MPX_EINVAL and b"null" in lib.mpx_last_error()
    rc = lib.mpx_rope_at(16, 16, 16, 16, st, st, 0, 8, 4, 128, None, 8, 2, 2, None, None)
    assert rc == _native.MPX_OK
    kst = (ctypes.c_int64 * 3)(8 * 4 * 128, 4 * 128, 128)
    rc = lib.mpx_kv_append_rope(16, 16, 16, 16, 16, 16, 16, kst, kst, 1, 8, 4, 128, 4, 16, 4, 2,
                                24, 16, 64, 2, 16, None)
    assert rc == _native.MPX_EINVAL and b"aligned" in lib.mpx_last_error()
    rc = lib.mpx_kv_append_rope(16, 16, 16, 16, 16, 16, 16, kst, kst, 1, 8, 4, 128, 4, 0, 4, 2,
                                16, 16, 64, 2, 16, None)
    assert rc == _native.MPX_EINVAL and b"block_size" in lib.mpx_last_error()
    rc = lib.mpx_kv_append_rope(16, 16, 16, 16, 16, 16, 16, kst, kst, 1, 8, 4, 128, 4, 16, 4, 5,
                                16, 16, 64, 2, 16, None)
    assert rc == _native.MPX_EINVAL and b"dtype" in lib.mpx_last_error()


def test_gqa_head_counts_validated(lib):
    st = (ctypes.c_int64 * 3)(8 * 64, 8 * 64, 64)
    rc = lib.mpx_attn_fwd_gqa(16, 16, 16, 16, st, st, st, st, 1, 6, 4, 8, 8, 64, 0.1, 1, -1, -1,
                              2, None, 0, None)
    assert rc == _native.MPX_EINVAL and b"multiple" in lib.mpx_last_error()
    st2 = (ctypes.c_int64 * 2)(4096, 128)
    rc = lib.mpx_paged_decode_gqa(16, 16, 16, 16, 16, None, 16, st2, st2, 1, 32, 5, 128, 4, 16,
                                  1, 0.1, 1, 16, 1 << 20, None)
    assert rc == _native.MPX_EINVAL and b"multiple" in lib.mpx_last_error()
    st3 = (ctypes.c_int64 * 3)(64 * 32 * 128, 128, 32 * 128)
    rc = lib.mpx_paged_prefill_gqa(16, 16, 16, 16, 16, None, 16, st3, st3, 1, 64, 32, 0, 128, 64,
                                   16, 8, 0.1, 1, 1, None, 0, None)
    assert rc == _native.MPX_EINVAL and b"multiple" in lib.mpx_last_error()


def _bwd(lib, dtype=2, D=64, B=1, H=2, H_kv=2, Sq=8, Sk=8, scale=0.1, ptr=16, ws=16,
         ws_bytes=1 << 20, stride=64):
    st = (ctypes.c_int64 * 3)(8 * 64 * H, 8 * 64, stride)
    return lib.mpx_attn_bwd(ptr, ptr, ptr, ptr, ptr, ptr, ptr, ptr, ptr, st, st, st, st, st, st,
                            st, st, B, H, H_kv, Sq, Sk, D, scale, 1, -1, -1, dtype, ws, ws_bytes,
                            None)


def _ds_blocks_brute(Sq, Sk, causal, wl, wr):
    """Stored-dS blocks of one head by brute force over the mask: key tile t
    (128 keys) keeps every 32-row query block from the first to the last one
    holding a query that sees one of its keys, times its four key blocks."""
    wr = 0 if causal else wr
    q = np.arange(Sq)[:, None]
    kk = np.arange(Sk)[None, :]
    vis = np.ones((Sq, Sk), bool)
    if wr >= 0:
        vis &= kk <= q + wr
    if wl >= 0:
        vis &= kk >= q - wl
    total = 0
    for t in range(0, Sk, 128):
        rows = np.nonzero(vis[:, t:t + 128].any(1))[0]
        if rows.size:
            total += 4 * (rows[-1] // 32 - rows[0] // 32 + 1)
    return total


@pytest.mark.parametrize("Sq,Sk,causal,wl,wr", [
    (4096, 4096, 1, -1, -1), (300, 77, 1, -1, -1), (77, 300, 0, -1, 223), (260, 260, 1, 75, -1),
    (260, 260, 0, 40, 40), (1, 129, 0, -1, -1), (129, 1, 1, -1, -1), (1000, 700, 0, 5, 900),
    (700, 1000, 0, 0, 0), (513, 513, 1, 127, -1)])
def test_bwd_ds_workspace_bytes(lib, Sq, Sk, causal, wl, wr):
    B, H = 2, 3
    dvec = (B * H * Sq * 4 + 255) // 256 * 256
    blocks = max(B * H * _ds_blocks_brute(Sq, Sk, causal, wl, wr), 2)
    for dtype in (1, 2):
        got = lib.mpx_attn_bwd_ds_workspace_bytes(B, H, Sq, Sk, 128, dtype, causal, wl, wr)
        assert got == dvec + 2048 * blocks
    # causal 4096: the 32 x 32 lower triangle (128 * 129 / 2 blocks) plus six unused
    # blocks on each key tile's diagonal
    if (Sq, Sk, causal) == (4096, 4096, 1):
        assert blocks == B * H * (128 * 129 // 2 + 6 * 32)
    # no stored-dS schedule: float32, head dims other than 128, empty problems
    assert lib.mpx_attn_bwd_ds_workspace_bytes(B, H, Sq, Sk, 128, 0, causal, wl, wr) == 0
    assert lib.mpx_attn_bwd_ds_workspace_bytes(B, H, Sq, Sk, 64, 2, causal, wl, wr) == 0
    assert lib.mpx_attn_bwd_ds_workspace_bytes(0, H, Sq, Sk, 128, 2, causal, wl, wr) == 0


def test_bwd_validation(lib):
    assert lib.mpx_attn_bwd_workspace_bytes(4, 32, 4096) == 4 * 32 * 4096 * 4
    assert lib.mpx_attn_bwd_workspace_bytes(0, 32, 4096) == 0
    assert _bwd(lib, stride=66, dtype=0) == _native.MPX_EINVAL  # f32: multiples of 4 elements
    assert _bwd(lib, dtype=9) == _native.MPX_EINVAL
    assert _bwd(lib, D=32) == _native.MPX_EUNSUPPORTED and b"head_dim" in lib.mpx_last_error()
    assert _bwd(lib, scale=-1.0) == _native.MPX_EINVAL and b"positive" in lib.mpx_last_error()
    assert _bwd(lib, H=6, H_kv=4) == _native.MPX_EINVAL and b"multiple" in lib.mpx_last_error()
    assert _bwd(lib, ptr=24) == _native.MPX_EINVAL and b"aligned" in lib.mpx_last_error()
    assert _bwd(lib, stride=68) == _native.MPX_EINVAL and b"multiples of 8" in lib.mpx_last_error()
    assert _bwd(lib, ws_bytes=8) == _native.MPX_EINVAL and b"workspace" in lib.mpx_last_error()
    assert _bwd(lib, ws=None) == _native.MPX_EINVAL and b"workspace" in lib.mpx_last_error()
    assert _bwd(lib, Sq=0, Sk=5) == _native.MPX_EINVAL and b"empty" in lib.mpx_last_error()
    assert _bwd(lib, B=0) == _native.MPX_OK and lib.mpx_last_error() == b""


def test_fwd_lse_validates_like_fwd(lib):
    st = (ctypes.c_int64 * 3)(8 * 64, 8 * 64, 64)
    rc = lib.mpx_attn_fwd_lse(16, 16, 16, 16, 16, st, st, st, st, 1, 1, 1, 8, 8, 96, 0.1, 1, -1,
                              -1, 2, None, 0, None)
    assert rc == _native.MPX_EUNSUPPORTED and b"head_dim" in lib.mpx_last_error()
    rc = lib.mpx_attn_fwd_lse(16, 16, 16, 16, None, st, st, st, st, 0, 1, 1, 8, 8, 64, 0.1, 1,
                              -1, -1, 2, None, 0, None)
    assert rc == _native.MPX_OK


def _fwd_rope(lib, dtype=2, cdt=2, q_offset=0, n_pos=8, ptr=16, cos=16, Sq=8):
    st = (ctypes.c_int64 * 3)(8 * 64, 8 * 64, 64)
    return lib.mpx_attn_fwd_rope(ptr, ptr, ptr, ptr, st, st, st, st, 1, 1, 1, Sq, 8, 64, 0.1, 1,
                                 -1, -1, dtype, cos, cos, q_offset, n_pos, cdt, None, 0, None)


def test_fwd_rope_validation(lib):
    assert _fwd_rope(lib, dtype=0) == _native.MPX_EUNSUPPORTED
    assert b"16-bit" in lib.mpx_last_error()
    assert _fwd_rope(lib, cdt=5) == _native.MPX_EINVAL and b"cache dtype" in lib.mpx_last_error()
    assert _fwd_rope(lib, q_offset=1) == _native.MPX_EINVAL and b"exceed" in lib.mpx_last_error()
    assert _fwd_rope(lib, cos=None) == _native.MPX_EINVAL and b"null" in lib.mpx_last_error()
    assert _fwd_rope(lib, cos=24) == _native.MPX_EINVAL and b"aligned" in lib.mpx_last_error()
    assert _fwd_rope(lib, Sq=0, cos=None) == _native.MPX_OK


def test_dropout_entries_validation(lib):
    st = (ctypes.c_int64 * 3)(8 * 64, 8 * 64, 64)

    def fwd(p=0.1, D=64, dtype=2, ptr=16, Sq=8):
        return lib.mpx_attn_fwd_dropout(ptr, ptr, ptr, ptr, None, st, st, st, st, 1, 1, 1, Sq, 8,
                                        D, 0.1, 1, -1, -1, dtype, p, 12345, None, 0, None)

    def bwd(p=0.1, D=64, scale=0.1):
        return lib.mpx_attn_bwd_dropout(*([16] * 9), *([st] * 8), 1, 1, 1, 8, 8, D, scale, 1, -1,
                                        -1, 2, p, 12345, 16, 1 << 20, None)

    for p in (1.0, -0.5, float("nan")):
        assert fwd(p=p) == _native.MPX_EINVAL and b"dropout_p" in lib.mpx_last_error()
        assert bwd(p=p) == _native.MPX_EINVAL and b"dropout_p" in lib.mpx_last_error()
    assert fwd(D=32) == _native.MPX_EUNSUPPORTED and b"64, 128" in lib.mpx_last_error()
    assert bwd(D=32) == _native.MPX_EUNSUPPORTED
    assert fwd(dtype=6) == _native.MPX_EINVAL and b"dtype" in lib.mpx_last_error()
    assert fwd(ptr=24) == _native.MPX_EINVAL and b"aligned" in lib.mpx_last_error()
    assert bwd(scale=-1.0) == _native.MPX_EINVAL and b"positive" in lib.mpx_last_error()
    assert fwd(Sq=0) == _native.MPX_OK  # empty problem: nothing enqueued

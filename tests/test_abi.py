"""C-ABI checks that need no GPU: the library loads, exports every function
declared in include/mpx_attn.h, and rejects bad arguments before any HIP call."""

import ctypes
import os
import re

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
        "mpx_paged_decode", "mpx_paged_decode_workspace_bytes"])


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

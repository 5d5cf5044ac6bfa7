"""Thread safety of the host layer (no GPU): the library loads once under
concurrent first calls, and mpx_last_error() is per thread, so concurrent
failing calls each read their own message. Counterpart of the reference's
stress tests (tests/stress/test_concurrency.py:150-345), which serialise MLX
behind a mutex; here no caller-side lock is needed.
"""

import concurrent.futures
import ctypes
import os
import threading

import pytest

from mlx_primitives import _native


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_native.library_path()):
        pytest.skip("libmpx_attn.so not built")
    return _native.load()


def test_concurrent_first_load(lib):
    saved = _native._lib
    try:
        _native._lib = None
        barrier = threading.Barrier(8)

        def first_load():
            barrier.wait()
            return _native.load()

        with concurrent.futures.ThreadPoolExecutor(max_workers=8) as ex:
            libs = list(ex.map(lambda _: first_load(), range(8)))
        assert all(x is libs[0] for x in libs)
    finally:
        _native._lib = saved


def test_error_messages_are_per_thread(lib):
    # Each thread makes a call that fails validation in its own way (nothing is
    # launched) and must read back its own message, many times, while the others do
    # the same.
    st = (ctypes.c_int64 * 3)(8 * 64, 8 * 64, 64)
    cases = {
        "dtype": lambda: lib.mpx_attn_fwd(16, 16, 16, 16, st, st, st, st, 1, 1, 8, 8, 64, 0.1, 1,
                                          -1, -1, 7, None, 0, None),
        "head_dim": lambda: lib.mpx_attn_fwd(16, 16, 16, 16, st, st, st, st, 1, 1, 8, 8, 96, 0.1,
                                             1, -1, -1, 2, None, 0, None),
        "aligned": lambda: lib.mpx_attn_fwd(18, 16, 16, 16, st, st, st, st, 1, 1, 8, 8, 64, 0.1, 1,
                                            -1, -1, 2, None, 0, None),
        "multiple": lambda: lib.mpx_attn_fwd_gqa(16, 16, 16, 16, st, st, st, st, 1, 6, 4, 8, 8,
                                                 64, 0.1, 1, -1, -1, 2, None, 0, None),
    }
    barrier = threading.Barrier(len(cases))

    def worker(word, call):
        barrier.wait()
        bad = 0
        for _ in range(2000):
            rc = call()
            msg = lib.mpx_last_error()
            if rc == 0 or word.encode() not in msg:
                bad += 1
        return bad

    with concurrent.futures.ThreadPoolExecutor(max_workers=len(cases)) as ex:
        futs = [ex.submit(worker, w, c) for w, c in cases.items()]
        assert [f.result() for f in futs] == [0] * len(cases)

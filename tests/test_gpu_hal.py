"""GPU tests of the run-time seam's copy contract (crates/tile_hal/src/buffer.rs:39-47):
the blocking th_memcpy_htod / th_memcpy_dtoh (cuda.rs:181-199 semantics) against
kernels on a non-blocking stream from th_stream_create, in both orders, through the
C ABI as the Rust binding in INTEGRATION.md calls it."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import tilers_hip as th
from tilers_hip._lib import check
from oracle import oracle as orc
from tests.tolerances import assert_softmax_close

pytestmark = pytest.mark.gpu

ROWS, COLS = 4096, 4096            # 64 MB of f32: the kernel runs long enough to race


def _malloc(dev, nbytes):
    p = C.c_void_p()
    check(th.lib().th_malloc(dev.handle, nbytes, C.byref(p)))
    return p.value


def test_blocking_htod_then_kernel_on_nonblocking_stream(dev):
    lib = th.lib()
    s = C.c_void_p()
    check(lib.th_stream_create(dev.handle, C.byref(s)))
    n = ROWS * COLS
    x = (np.random.default_rng(7).standard_normal(n) * 2).astype(np.float32)
    px, py = _malloc(dev, n * 4), _malloc(dev, n * 4)
    try:
        # copy on the null stream, blocking: done when it returns ...
        check(lib.th_memcpy_htod(px, x.ctypes.data, n * 4))
        # ... so a kernel on the non-blocking stream reads the new data
        check(lib.th_softmax(px, py, ROWS, COLS, int(th.TileDtype.F32), s.value))
        check(lib.th_stream_sync(s.value))
        y = np.empty(n, np.float32)
        check(lib.th_memcpy_dtoh(y.ctypes.data, py, n * 4))
        rows = slice(0, 64)
        ref = orc.softmax(x.reshape(ROWS, COLS)[rows], 64, COLS)
        assert_softmax_close(y.reshape(ROWS, COLS)[rows], ref, "softmax after blocking htod")
        assert np.allclose(y.reshape(ROWS, COLS).astype(np.float64).sum(axis=1), 1.0, atol=1e-4)
    finally:
        check(lib.th_free(dev.handle, px))
        check(lib.th_free(dev.handle, py))
        check(lib.th_stream_destroy(s.value))


def test_kernel_on_nonblocking_stream_then_blocking_dtoh(dev):
    lib = th.lib()
    s = C.c_void_p()
    check(lib.th_stream_create(dev.handle, C.byref(s)))
    n = ROWS * COLS
    p = _malloc(dev, n * 4)
    try:
        check(lib.th_memset_async(p, 0, n * 4, s.value))
        for seed in (11, 12):   # the second fill must be what the copy sees
            check(lib.th_fill_random(p, n, int(th.TileDtype.F32), 1, 0.0, 1.0, seed, s.value))
        # the binding drains the caller's stream, then copies (blocking)
        check(lib.th_stream_sync(s.value))
        got = np.empty(n, np.float32)
        check(lib.th_memcpy_dtoh(got.ctypes.data, p, n * 4))
        # the same fill through the asynchronous copy on the same stream
        ref = np.empty(n, np.float32)
        check(lib.th_fill_random(p, n, int(th.TileDtype.F32), 1, 0.0, 1.0, 12, s.value))
        check(lib.th_memcpy_dtoh_async(ref.ctypes.data, p, n * 4, s.value))
        check(lib.th_stream_sync(s.value))
        assert np.array_equal(got, ref)
        assert np.count_nonzero(got) > n // 2
    finally:
        check(lib.th_free(dev.handle, p))
        check(lib.th_stream_destroy(s.value))


def test_blocking_copies_zero_bytes_are_noops():
    lib = th.lib()
    assert lib.th_memcpy_htod(None, None, 0) == 0
    assert lib.th_memcpy_dtoh(None, None, 0) == 0

"""th_attention_decode_static (the decode entry point that allocates nothing)
against th_attention_decode through the C ABI: bit-identical outputs on two
calls in a row, the second with a smaller input, including shapes that split
the KV sequence (partials in the fixed per-GPU scratch array)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import tilers_hip as th
from tilers_hip._lib import check

pytestmark = pytest.mark.gpu

D = th.TileDtype


def _decode_pair(dev, stream, B, L, max_seq, NH, NKV, dtype, seed, Dh=128):
    nq, nkv = B * NH * Dh, B * NKV * max_seq * Dh
    bufs = [dev.alloc(n, dtype) for n in (nq, nkv, nkv)]
    for i, (b, n) in enumerate(zip(bufs, (nq, nkv, nkv))):
        th.fill_random(b, n, dtype, "normal", 0.0, 1.0, seed + i, stream)
    q, k, v = bufs
    o_ref, o_static = dev.alloc(nq, dtype), dev.alloc(nq, dtype)
    # non-zero garbage in the outputs: the static path must overwrite all of it
    th.fill_random(o_static, nq, dtype, "uniform", 5.0, 6.0, seed + 9, stream)
    wsz = th.attention_decode_workspace_size(B, L, Dh, NH, NKV)
    ws = dev.alloc(max(1, wsz // 4), D.F32)
    th.attention_decode(q, k, v, o_ref, B, L, max_seq, Dh, NH, NKV, dtype, ws, wsz, stream)
    rc = th.lib().th_attention_decode_static(
        C.c_void_p(q.as_raw_ptr()), C.c_void_p(k.as_raw_ptr()), C.c_void_p(v.as_raw_ptr()),
        C.c_void_p(o_static.as_raw_ptr()), B, L, max_seq, Dh, NH, NKV, int(dtype), stream.handle)
    check(rc)
    a, b = o_ref.copy_to_host(stream), o_static.copy_to_host(stream)
    return a, b


@pytest.mark.parametrize("dtype", [D.BF16, D.F16])
def test_decode_static_matches_decode_two_calls(dev, stream, dtype):
    # first call: B=1, L=20000 -> 2 items, about 40 splits: partials in the scratch
    a, b = _decode_pair(dev, stream, 1, 20000, 20011, 8, 2, dtype, 0x5eed0)
    assert np.isfinite(a.astype(np.float32) if a.dtype != np.uint16 else a).all()
    assert np.array_equal(a, b)
    # second call, smaller: fewer partials, different grouping (G=1, 4 heads)
    a, b = _decode_pair(dev, stream, 1, 3000, 3000, 4, 4, dtype, 0x5eed1)
    assert np.array_equal(a, b)


def test_decode_static_unsplit_and_empty(dev, stream):
    # 512 items: one workgroup per item, no partials (the scratch is not touched)
    a, b = _decode_pair(dev, stream, 64, 700, 700, 8, 8, D.BF16, 0x5eed2)
    assert np.array_equal(a, b)
    # seq_len 0: zeros, written by a kernel
    o = dev.alloc(2 * 4 * 128, D.BF16)
    th.fill_random(o, 2 * 4 * 128, D.BF16, "uniform", 1.0, 2.0, 3, stream)
    q = dev.alloc(2 * 4 * 128, D.BF16)
    kv = dev.alloc(2 * 4 * 16 * 128, D.BF16)
    check(th.lib().th_attention_decode_static(
        C.c_void_p(q.as_raw_ptr()), C.c_void_p(kv.as_raw_ptr()), C.c_void_p(kv.as_raw_ptr()),
        C.c_void_p(o.as_raw_ptr()), 2, 0, 16, 128, 4, 4, int(D.BF16), stream.handle))
    assert not o.copy_to_host(stream).any()


def test_decode_static_head_dim_64(dev, stream):
    """head_dim 64 runs natively (no padded copies), so the static entry serves it."""
    a, b = _decode_pair(dev, stream, 1, 9000, 9000, 8, 2, D.BF16, 0x5eed3, Dh=64)
    assert np.array_equal(a, b)
    a, b = _decode_pair(dev, stream, 2, 500, 512, 4, 4, D.BF16, 0x5eed4, Dh=64)
    assert np.array_equal(a, b)


def test_decode_static_general_shapes(dev, stream):
    """Shapes th_attention_decode runs on the general kernel (no scratch): the static
    entry serves them too.  head_dim 96 with 3 query heads per kv head is not padded
    (the MFMA decode takes groups of 1, 2, 4, 8 or 16)."""
    a, b = _decode_pair(dev, stream, 2, 700, 704, 6, 2, D.BF16, 0x5eed5, Dh=96)
    assert np.array_equal(a, b)
    a, b = _decode_pair(dev, stream, 1, 300, 300, 3, 1, D.F16, 0x5eed6, Dh=96)
    assert np.array_equal(a, b)


def test_decode_static_rejects_padded_head_dim(dev, stream):
    q = dev.alloc(4 * 96, D.BF16)
    kv = dev.alloc(4 * 64 * 96, D.BF16)
    rc = th.lib().th_attention_decode_static(
        C.c_void_p(q.as_raw_ptr()), C.c_void_p(kv.as_raw_ptr()), C.c_void_p(kv.as_raw_ptr()),
        C.c_void_p(q.as_raw_ptr()), 1, 64, 64, 96, 4, 4, int(D.BF16), stream.handle)
    assert rc != 0
    assert b"padded" in th.lib().th_last_error()

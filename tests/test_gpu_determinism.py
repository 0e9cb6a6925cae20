"""Repeated launches on the same inputs give the same bits (MI355X only).

Every kernel here fixes its summation order (no atomics in the data path, split
partials merged in index order), so a launch-to-launch difference can only come from
a race or a missing wait state.  Such a fault can stay inside the parity tolerances
(the prefill loop's once did: 1-2 ulp on 1.6% of config-4 outputs), so each op runs
three times at a BASELINE shape, or a shape that takes its split and streaming paths,
and all outputs must match launch 0 exactly.
"""
from __future__ import annotations

import numpy as np
import pytest

import tilers_hip as th

pytestmark = pytest.mark.gpu

D = th.TileDtype


def rnd(dev, stream, n, dtype, seed, dist="normal", p0=0.0, p1=1.0):
    buf = dev.alloc(n, dtype)
    th.fill_random(buf, n, dtype, dist, p0, p1, seed, stream)
    return buf


def same_bits(run, out, stream, reps=3):
    first = None
    for i in range(reps):
        run()
        got = out.copy_to_host(stream).copy()
        if first is None:
            first = got
        else:
            nd = int(np.count_nonzero(got.view(np.uint8) != first.view(np.uint8)))
            assert nd == 0, f"launch {i}: {nd} bytes differ from launch 0"


def test_softmax_config1(dev, stream):
    rows, cols = 8192, 1024
    x = rnd(dev, stream, rows * cols, D.F32, 0xD1, p1=2.0)
    y = dev.alloc(rows * cols, D.F32)
    same_bits(lambda: th.softmax(x, y, rows, cols, D.F32, stream), y, stream)


def test_softmax_chunked_rows(dev, stream):
    """64 rows of 131072: chunk statistics merged per row (two kernels)."""
    rows, cols = 64, 131072
    x = rnd(dev, stream, rows * cols, D.F32, 0xD2, p1=2.0)
    y = dev.alloc(rows * cols, D.F32)
    same_bits(lambda: th.softmax(x, y, rows, cols, D.F32, stream), y, stream)


def test_matmul_config2(dev, stream):
    n = 4096
    a = rnd(dev, stream, n * n, D.BF16, 0xD3, "uniform", -1.0, 1.0)
    b = rnd(dev, stream, n * n, D.BF16, 0xD4, "uniform", -1.0, 1.0)
    c = dev.alloc(n * n, D.F32)
    same_bits(lambda: th.matmul(a, b, c, n, n, n, D.BF16, D.F32, stream=stream), c, stream)


def test_matmul_split_k(dev, stream):
    """M=8: split-K slices reduced in order."""
    m, k, n = 8, 14336, 4096
    a = rnd(dev, stream, m * k, D.BF16, 0xD5)
    b = rnd(dev, stream, n * k, D.BF16, 0xD6, p1=0.02)
    c = dev.alloc(m * n, D.BF16)
    same_bits(lambda: th.matmul(a, b, c, m, k, n, D.BF16, D.BF16, True, stream=stream), c,
              stream)


def test_matmul_silu_mul(dev, stream):
    m, k, n = 1024, 4096, 2048
    a = rnd(dev, stream, m * k, D.F16, 0xD7)
    b = rnd(dev, stream, k * n, D.F16, 0xD8, p1=0.02)
    up = rnd(dev, stream, m * n, D.F16, 0xD9)
    c = dev.alloc(m * n, D.F16)
    same_bits(lambda: th.matmul_silu_mul(a, b, up, c, m, k, n, D.F16, D.F16, stream=stream), c,
              stream)


def test_matmul_f32_mfma(dev, stream):
    n = 1024
    a = rnd(dev, stream, n * n, D.F32, 0xDA)
    b = rnd(dev, stream, n * n, D.F32, 0xDB)
    c = dev.alloc(n * n, D.F32)
    same_bits(lambda: th.matmul(a, b, c, n, n, n, D.F32, D.F32, stream=stream), c, stream)


def test_rms_norm(dev, stream):
    rows, cols = 8192, 4096
    x = rnd(dev, stream, rows * cols, D.BF16, 0xDC)
    y = dev.alloc(rows * cols, D.BF16)
    same_bits(lambda: th.rms_norm(x, y, rows, cols, 1e-6, D.BF16, stream), y, stream)


def test_attention_f32(dev, stream):
    s, d, tiles = 2048, 128, 4
    q, k, v = (rnd(dev, stream, tiles * s * d, D.F32, 0xDD + i) for i in range(3))
    o = dev.alloc(tiles * s * d, D.F32)
    same_bits(lambda: th.attention(q, k, v, o, s, d, tiles, D.F32, stream), o, stream)


@pytest.mark.parametrize("B,L,NH,NKV", [(64, 8192, 32, 8), (1, 32768, 32, 8)])
def test_decode(dev, stream, B, L, NH, NKV):
    """Config 5 (unsplit), and B=1 L=32K (64-way split merged by the combine kernel)."""
    Dh = 128
    q = rnd(dev, stream, B * NH * Dh, D.BF16, 0xE0)
    k = rnd(dev, stream, B * NKV * L * Dh, D.BF16, 0xE1)
    v = rnd(dev, stream, B * NKV * L * Dh, D.BF16, 0xE2)
    o = dev.alloc(B * NH * Dh, D.BF16)
    same_bits(lambda: th.attention_decode(q, k, v, o, B, L, L, Dh, NH, NKV, D.BF16, stream=stream),
              o, stream)


def test_prefill_gqa_chunk(dev, stream):
    """GQA 4:1 chunked prefill (start_pos > 0), grouped work order."""
    B, S, start, NH, NKV, Dh = 2, 1000, 700, 32, 8, 128
    max_seq = start + S
    q = rnd(dev, stream, B * S * NH * Dh, D.BF16, 0xE3)
    k = rnd(dev, stream, B * NKV * max_seq * Dh, D.BF16, 0xE4)
    v = rnd(dev, stream, B * NKV * max_seq * Dh, D.BF16, 0xE5)
    o = dev.alloc(B * S * NH * Dh, D.BF16)
    same_bits(lambda: th.attention_prefill(q, k, v, o, B, S, start, max_seq, Dh, NH, NKV, D.BF16,
                                           stream), o, stream)


def test_prefill_split_kv(dev, stream):
    """A 512-token chunk after 7680 cached positions: split-KV parts and their merge."""
    B, S, start, NH, NKV, Dh = 1, 512, 7680, 32, 8, 128
    max_seq = start + S
    q = rnd(dev, stream, B * S * NH * Dh, D.BF16, 0xE6)
    k = rnd(dev, stream, B * NKV * max_seq * Dh, D.BF16, 0xE7)
    v = rnd(dev, stream, B * NKV * max_seq * Dh, D.BF16, 0xE8)
    o = dev.alloc(B * S * NH * Dh, D.BF16)
    same_bits(lambda: th.attention_prefill(q, k, v, o, B, S, start, max_seq, Dh, NH, NKV, D.BF16,
                                           stream), o, stream)


def test_prefill_head_dim_64(dev, stream):
    B, S, NH, NKV, Dh = 2, 2048, 16, 4, 64
    q = rnd(dev, stream, B * S * NH * Dh, D.BF16, 0xE9)
    k = rnd(dev, stream, B * NKV * S * Dh, D.BF16, 0xEA)
    v = rnd(dev, stream, B * NKV * S * Dh, D.BF16, 0xEB)
    o = dev.alloc(B * S * NH * Dh, D.BF16)
    same_bits(lambda: th.attention_prefill(q, k, v, o, B, S, 0, S, Dh, NH, NKV, D.BF16, stream), o,
              stream)

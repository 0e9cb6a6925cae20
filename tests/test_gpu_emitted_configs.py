"""BASELINE's five configurations through the unchanged tile_std path: MLIR ->
th_emit (the `hip` CodegenTarget) -> gfx950 code object -> th_launcher_launch,
compared with the CPU oracle on every output element (config 4 against the
session-wide oracle result of tests/conftest.py, shared with the library test)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import tilers_hip as th
from oracle import oracle as orc
from tests.tolerances import assert_attn_close, assert_gemm_close, assert_softmax_close
from tilers_hip import _build

pytestmark = pytest.mark.gpu
D = th.TileDtype
SEED0 = 0x71130000


@pytest.fixture(scope="module")
def launcher(dev):
    lau = dev.create_launcher()
    for stem in ("softmax_rows", "config_gemms", "prefill_bf16", "decode_bf16"):
        lau.load(_build.example_path(stem), th.KernelMode.GENERAL)
    return lau


def ptr(b):
    return C.c_void_p(b.as_raw_ptr())


def rnd(dev, stream, n, dtype, dist, p0, p1, seed):
    b = dev.alloc(n, dtype)
    th.fill_random(b, n, dtype, dist, p0, p1, seed, stream)
    return b


def test_config1_softmax_emitted(dev, stream, launcher):
    rows, cols = 8192, 1024          # 8192 logical 1 x 1024 tiles
    x = rnd(dev, stream, rows * cols, D.F32, "normal", 0.0, 2.0, SEED0 + 1)
    y = dev.alloc(rows * cols, D.F32)
    launcher.launch("softmax_rows_f32", th.LaunchGrid.cuda(rows, cols), [ptr(x), ptr(y)], stream)
    xh = x.copy_to_host(stream).reshape(rows, cols)
    assert_softmax_close(y.copy_to_host(stream).reshape(rows, cols), orc.softmax(xh, rows, cols),
                         "emitted config1")


def test_config2_gemm_emitted(dev, stream, launcher):
    M = N = K = 4096
    a = rnd(dev, stream, M * K, D.BF16, "uniform", -1.0, 1.0, SEED0 + 2)
    b = rnd(dev, stream, K * N, D.BF16, "uniform", -1.0, 1.0, SEED0 + 102)
    c = dev.alloc(M * N, D.F32)
    launcher.launch("gemm_4096_bf16_acc_f32", th.LaunchGrid.blocks_only(1), [ptr(a), ptr(b), ptr(c)],
                    stream)
    ref = orc.matmul(a.copy_to_host(stream), b.copy_to_host(stream), M, K, N, orc.BF16)
    assert_gemm_close(c.copy_to_host(stream).reshape(M, N), ref.reshape(M, N), "emitted config2")


def test_config3_mlp_emitted(dev, stream, launcher):
    M, K, N = 8192, 4096, 14336
    a = rnd(dev, stream, M * K, D.F16, "normal", 0.0, 1.0, SEED0 + 3)
    b = rnd(dev, stream, K * N, D.F16, "normal", 0.0, 0.02, SEED0 + 103)
    c = dev.alloc(M * N, D.F16)
    launcher.launch("mlp_up_f16", th.LaunchGrid.blocks_only(1), [ptr(a), ptr(b), ptr(c)], stream)
    ref = orc.matmul(a.copy_to_host(stream), b.copy_to_host(stream), M, K, N, orc.F16, orc.F32)
    got = orc.widen(c.copy_to_host(stream), orc.F16).reshape(M, N)
    assert_gemm_close(got, orc.widen(orc.narrow(ref, orc.F16), orc.F16).reshape(M, N),
                      "emitted config3", u16_dtype=orc.F16)


def test_config3_swiglu_emitted(dev, stream, launcher):
    """Config 3's shape with the gate epilogue through the emitter (the assembly entry's
    SiLU*Mul program): 96 rows against the oracle."""
    M, K, N = 8192, 4096, 14336
    a = rnd(dev, stream, M * K, D.F16, "normal", 0.0, 1.0, SEED0 + 3)
    b = rnd(dev, stream, K * N, D.F16, "normal", 0.0, 0.02, SEED0 + 103)
    u = rnd(dev, stream, M * N, D.F16, "normal", 0.0, 1.0, SEED0 + 203)
    c = dev.alloc(M * N, D.F16)
    launcher.launch("mlp_gate_f16", th.LaunchGrid.blocks_only(1), [ptr(a), ptr(b), ptr(u), ptr(c)],
                    stream)
    ah = a.copy_to_host(stream).reshape(M, K)
    bh, uh = b.copy_to_host(stream), u.copy_to_host(stream).reshape(M, N)
    got = orc.widen(c.copy_to_host(stream), orc.F16).reshape(M, N)
    for r0 in (0, 4064, 8160):
        ref = orc.matmul_silu_mul(np.ascontiguousarray(ah[r0:r0 + 32]), bh,
                                  np.ascontiguousarray(uh[r0:r0 + 32]), 32, K, N, orc.F16, orc.F16)
        assert_gemm_close(got[r0:r0 + 32], orc.widen(ref, orc.F16).reshape(32, N),
                          f"emitted config3 swiglu rows {r0}", u16_dtype=orc.F16)


def test_config4_prefill_emitted(dev, stream, launcher, config4):
    c = config4                        # batch = logical tiles
    o = dev.alloc(c.n, D.BF16)
    scal = [C.c_uint32(x) for x in (c.S, 0, c.S, c.Dh, c.H, c.H)]
    args = [ptr(c.q), ptr(c.k), ptr(c.v), ptr(o)] + scal
    # one 512-thread workgroup per (batch, head, 256-query block), as the library launches
    assert launcher.hardware_grid("prefill_bf16", th.LaunchGrid.blocks_only(c.B), args) == \
        (c.B * c.H * c.S // 256, 512)
    launcher.launch("prefill_bf16", th.LaunchGrid.blocks_only(c.B), args, stream)
    got = orc.widen(o.copy_to_host(stream), orc.BF16).reshape(c.B, c.S, c.H, c.Dh)
    assert np.isfinite(got).all()
    for b in range(c.B):
        assert_attn_close(got[b], c.ref[b], f"emitted config4 batch {b}")


def test_config5_decode_emitted(dev, stream, launcher):
    B, NH, NKV, L, Dh = 64, 32, 8, 8192, 128
    q = rnd(dev, stream, B * NH * Dh, D.BF16, "normal", 0.0, 1.0, SEED0 + 5)
    k = rnd(dev, stream, B * NKV * L * Dh, D.BF16, "normal", 0.0, 1.0, SEED0 + 105)
    v = rnd(dev, stream, B * NKV * L * Dh, D.BF16, "normal", 0.0, 1.0, SEED0 + 205)
    o = dev.alloc(B * NH * Dh, D.BF16)
    scal = [C.c_uint32(x) for x in (L, L, Dh, NH, NKV)]
    args = [ptr(q), ptr(k), ptr(v), ptr(o)] + scal
    # two workgroups per CU; 512 (batch, kv_head) items on MI355X's 256 CUs run unsplit
    grid, threads = launcher.hardware_grid("decode_bf16", th.LaunchGrid.blocks_only(B), args)
    assert threads == 256 and grid == min(B * NKV * (L // 512), 2 * dev.cu_count())
    launcher.launch("decode_bf16", th.LaunchGrid.blocks_only(B), args, stream)
    ref = orc.attention_decode(q.copy_to_host(stream), k.copy_to_host(stream),
                               v.copy_to_host(stream), orc.BF16, B, L, L, Dh, NH, NKV)
    assert_attn_close(orc.widen(o.copy_to_host(stream), orc.BF16), ref, "emitted config5")


def test_decode_long_context_splits_in_kernel(dev, stream, launcher):
    """B = 1, L = 32K: 8 (batch, kv_head) items over a grid of two workgroups per CU.
    Each item's 64 chunks are split over 64 workgroups and the last to finish merges
    the partials; a second launch (arrival counters reset by the first) gives the same
    bits."""
    B, NH, NKV, L, Dh = 1, 32, 8, 32768, 128
    q = rnd(dev, stream, B * NH * Dh, D.BF16, "normal", 0.0, 1.0, SEED0 + 6)
    k = rnd(dev, stream, B * NKV * L * Dh, D.BF16, "normal", 0.0, 1.0, SEED0 + 106)
    v = rnd(dev, stream, B * NKV * L * Dh, D.BF16, "normal", 0.0, 1.0, SEED0 + 206)
    o = dev.alloc(B * NH * Dh, D.BF16)
    scal = [C.c_uint32(x) for x in (L, L, Dh, NH, NKV)]
    args = [ptr(q), ptr(k), ptr(v), ptr(o)] + scal
    grid, _ = launcher.hardware_grid("decode_bf16", th.LaunchGrid.blocks_only(B), args)
    assert grid == min(NKV * (L // 512), 2 * dev.cu_count()) and grid > B * NKV
    launcher.launch("decode_bf16", th.LaunchGrid.blocks_only(B), args, stream)
    first = o.copy_to_host(stream)
    ref = orc.attention_decode(q.copy_to_host(stream), k.copy_to_host(stream),
                               v.copy_to_host(stream), orc.BF16, B, L, L, Dh, NH, NKV)
    assert_attn_close(orc.widen(first, orc.BF16), ref, "emitted decode B=1 L=32K")
    launcher.launch("decode_bf16", th.LaunchGrid.blocks_only(B), args, stream)
    np.testing.assert_array_equal(o.copy_to_host(stream), first)


@pytest.mark.parametrize("B,L,max_seq", [(1, 40000, 40003), (3, 513, 600), (1, 1, 8)])
def test_decode_split_ragged(dev, stream, launcher, B, L, max_seq):
    """79 chunks over 4 items: 40 splits of two chunks, the last of one; two chunks
    with a one-position last chunk; a single position (nothing to split)."""
    NH, NKV, Dh = 16, 4, 128
    q = rnd(dev, stream, B * NH * Dh, D.BF16, "normal", 0.0, 1.0, SEED0 + 7 + L)
    k = rnd(dev, stream, B * NKV * max_seq * Dh, D.BF16, "normal", 0.0, 1.0, SEED0 + 107 + L)
    v = rnd(dev, stream, B * NKV * max_seq * Dh, D.BF16, "normal", 0.0, 1.0, SEED0 + 207 + L)
    o = dev.alloc(B * NH * Dh, D.BF16)
    scal = [C.c_uint32(x) for x in (L, max_seq, Dh, NH, NKV)]
    launcher.launch("decode_bf16", th.LaunchGrid.blocks_only(B), [ptr(q), ptr(k), ptr(v), ptr(o)] + scal,
                    stream)
    ref = orc.attention_decode(q.copy_to_host(stream), k.copy_to_host(stream),
                               v.copy_to_host(stream), orc.BF16, B, L, max_seq, Dh, NH, NKV)
    assert_attn_close(orc.widen(o.copy_to_host(stream), orc.BF16), ref, f"emitted decode B={B} L={L}")

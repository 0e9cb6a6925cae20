"""Kernels emitted by the `hip` target, launched through the HAL launcher.

The example modules (tile-rs_amd/tilers_hip/examples/*.mlir) are emitted and
compiled to gfx950 code objects by build(); here each is loaded with
hipModuleLoad, launched by name on a 1-D grid of logical tiles (the launch
descriptor expands it to the hardware grid), and compared with the CPU oracle.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import tilers_hip as th
from oracle import oracle as orc
from tests.tolerances import (assert_attn_close, assert_gemm_close, assert_softmax_close,
                              assert_within_ulp16, ulp16)
from tilers_hip import _build

pytestmark = pytest.mark.gpu
D = th.TileDtype


@pytest.fixture(scope="module")
def launcher(dev):
    lau = dev.create_launcher()
    for stem in ("softmax_rows", "softmax_generic", "matmul_bf16", "matmul_f16_t", "matmul_f32",
                 "attention_f32", "prefill_bf16", "decode_bf16", "swiglu_mask", "rms_norm_rows",
                 "swiglu_gate_bf16", "matmul_bf16_tiles", "rope", "rows_long", "ops_extra",
                 "softmax_loop", "softmax_loop_generic", "gemm_loop", "attention_gqa"):
        lau.load(_build.example_path(stem), th.KernelMode.GENERAL)
    return lau


def up(dev, s, a, dt):
    b = dev.alloc(a.size, dt)
    b.copy_from_host(np.ascontiguousarray(a).reshape(-1), s)
    return b


def ptr(b):
    return C.c_void_p(b.as_raw_ptr())


def test_softmax_rows_f32(dev, stream, launcher):
    tiles = 300  # 1 x 1024 tiles, grid = tiles (the #[tile_kernel] launch shape)
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((tiles, 1024)) * 2).astype(np.float32)
    xb, yb = up(dev, stream, x, D.F32), dev.alloc(x.size, D.F32)
    launcher.launch("softmax_rows_f32", th.LaunchGrid.cuda(tiles, 1024), [ptr(xb), ptr(yb)], stream)
    assert_softmax_close(yb.copy_to_host(stream).reshape(tiles, 1024), orc.softmax(x, tiles, 1024))


def test_long_rows_one_workgroup_per_row(dev, stream, launcher):
    """Emitted softmax over 1 x 16384 f32 tiles and RMSNorm over 2 x 8192 f32 tiles: one
    workgroup per row, the row in registers."""
    rng = np.random.default_rng(43)
    tiles = 37
    x = (rng.standard_normal((tiles, 16384)) * 2).astype(np.float32)
    xb, yb = up(dev, stream, x, D.F32), dev.alloc(x.size, D.F32)
    launcher.launch("softmax_long_f32", th.LaunchGrid.blocks_only(tiles), [ptr(xb), ptr(yb)], stream)
    assert_softmax_close(yb.copy_to_host(stream).reshape(tiles, 16384), orc.softmax(x, tiles, 16384))
    x2 = rng.standard_normal((tiles * 2, 8192)).astype(np.float32)
    xb2, yb2 = up(dev, stream, x2, D.F32), dev.alloc(x2.size, D.F32)
    launcher.launch("rms_long_f32", th.LaunchGrid.blocks_only(tiles), [ptr(xb2), ptr(yb2)], stream)
    assert_softmax_close(yb2.copy_to_host(stream).reshape(tiles * 2, 8192),
                         orc.rms_norm(x2, tiles * 2, 8192, 1e-5))


def test_rope_f32(dev, stream, launcher):
    """__tile_rope_f32 on 4 x 64 tiles at pos 7 against the oracle (mlir_to_gpu.rs:1508-1557).
    Frequency and angle are f32 on both sides; powf/cosf/sinf may differ by an ulp or
    two, which moves the output by < 1e-6 here."""
    tiles = 50
    rng = np.random.default_rng(41)
    x = rng.standard_normal((tiles * 4, 64)).astype(np.float32)
    xb, yb = up(dev, stream, x, D.F32), dev.alloc(x.size, D.F32)
    launcher.launch("rope_f32", th.LaunchGrid.blocks_only(tiles), [ptr(xb), ptr(yb)], stream)
    got = yb.copy_to_host(stream).reshape(tiles * 4, 64)
    ref = orc.rope(x, tiles * 4, 64, 7)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_rope_bf16_large_position(dev, stream, launcher):
    """__tile_rope_f16 with a bf16 name, 2 x 128 tiles at pos 1000.  At this position a
    one-ulp difference in the f32 frequency moves the angle by up to 6e-5 rad, so the
    bound is one bf16 ulp plus 2.5e-4 per unit of the pair's magnitude."""
    tiles = 20
    rng = np.random.default_rng(42)
    x = orc.narrow(rng.standard_normal(tiles * 2 * 128).astype(np.float32), orc.BF16)
    xb, yb = up(dev, stream, x, D.BF16), dev.alloc(x.size, D.BF16)
    launcher.launch("rope_bf16", th.LaunchGrid.blocks_only(tiles), [ptr(xb), ptr(yb)], stream)
    got = orc.widen(yb.copy_to_host(stream), orc.BF16).astype(np.float64)
    ref = orc.widen(orc.rope(x, tiles * 2, 128, 1000, orc.BF16), orc.BF16).astype(np.float64)
    xw = orc.widen(x, orc.BF16).astype(np.float64).reshape(-1, 2)
    mag = np.repeat(np.abs(xw).sum(axis=1), 2)
    bad = np.abs(got - ref) > ulp16(ref, orc.BF16) + 2.5e-4 * mag
    assert not bad.any(), (np.flatnonzero(bad)[:8], got[bad][:8], ref[bad][:8])


def test_softmax_generic_form_bf16(dev, stream, launcher):
    tiles = 3  # 4 x 2048 tiles
    rng = np.random.default_rng(2)
    x = orc.narrow((rng.standard_normal(tiles * 4 * 2048) * 2).astype(np.float32), orc.BF16)
    xb, yb = up(dev, stream, x, D.BF16), dev.alloc(x.size, D.BF16)
    launcher.launch("softmax_bf16_generic", th.LaunchGrid.blocks_only(tiles), [ptr(xb), ptr(yb)], stream)
    got = orc.widen(yb.copy_to_host(stream), orc.BF16)
    ref = orc.softmax(orc.widen(x, orc.BF16), tiles * 4, 2048)
    assert_within_ulp16(got, ref.reshape(-1), orc.BF16)


def test_matmul_bf16_acc_f32_two_tiles(dev, stream, launcher):
    tiles, M, K, N = 2, 512, 256, 384
    rng = np.random.default_rng(3)
    a = orc.narrow(rng.uniform(-1, 1, tiles * M * K).astype(np.float32), orc.BF16)
    b = orc.narrow(rng.uniform(-1, 1, tiles * K * N).astype(np.float32), orc.BF16)
    ab, bb, cb = up(dev, stream, a, D.BF16), up(dev, stream, b, D.BF16), dev.alloc(tiles * M * N, D.F32)
    launcher.launch("matmul_bf16_acc_f32", th.LaunchGrid.blocks_only(tiles), [ptr(ab), ptr(bb), ptr(cb)],
                    stream)
    got = cb.copy_to_host(stream).reshape(tiles, M, N)
    for t in range(tiles):
        ref = orc.matmul(a[t * M * K:(t + 1) * M * K], b[t * K * N:(t + 1) * K * N], M, K, N, orc.BF16)
        assert_gemm_close(got[t], ref, f"tile {t}")


@pytest.mark.parametrize("c_shift", [0, 2])
def test_matmul_bf16_whole_tiles(dev, stream, launcher, c_shift):
    """512x320x768 bf16 -> bf16 over two logical tiles: the LDS-DMA entry.  With C two
    bytes past a 16-byte boundary the entry takes its per-element kernel instead."""
    tiles, M, K, N = 2, 512, 320, 768
    rng = np.random.default_rng(5 + c_shift)
    a = orc.narrow(rng.standard_normal(tiles * M * K).astype(np.float32), orc.BF16)
    b = orc.narrow((rng.standard_normal(tiles * K * N) * 0.05).astype(np.float32), orc.BF16)
    ab, bb = up(dev, stream, a, D.BF16), up(dev, stream, b, D.BF16)
    cb = dev.alloc(tiles * M * N + 8, D.BF16)
    launcher.launch("matmul_bf16_tiles", th.LaunchGrid.blocks_only(tiles),
                    [ptr(ab), ptr(bb), C.c_void_p(cb.as_raw_ptr() + c_shift)], stream)
    raw = cb.copy_to_host(stream)[c_shift // 2:c_shift // 2 + tiles * M * N]
    got = orc.widen(raw, orc.BF16).reshape(tiles, M, N)
    for t in range(tiles):
        ref = orc.matmul(a[t * M * K:(t + 1) * M * K], b[t * K * N:(t + 1) * K * N], M, K, N,
                         orc.BF16, orc.F32)
        assert_gemm_close(got[t], orc.widen(orc.narrow(ref, orc.BF16), orc.BF16),
                          f"matmul_bf16_tiles tile {t} shift {c_shift}", u16_dtype=orc.BF16)


def test_matmul_transposed_f16_out(dev, stream, launcher):
    M, K, N = 128, 320, 264
    rng = np.random.default_rng(4)
    a = orc.narrow(rng.standard_normal(M * K).astype(np.float32), orc.F16)
    b = orc.narrow((rng.standard_normal(N * K) * 0.02).astype(np.float32), orc.F16)
    ab, bb, cb = up(dev, stream, a, D.F16), up(dev, stream, b, D.F16), dev.alloc(M * N, D.F16)
    launcher.launch("matmul_t_f16", th.LaunchGrid.blocks_only(1), [ptr(ab), ptr(bb), ptr(cb)], stream)
    got = orc.widen(cb.copy_to_host(stream), orc.F16).reshape(M, N)
    ref = orc.matmul(a, b, M, K, N, orc.F16, orc.F32, b_trans=True)
    assert_gemm_close(got, orc.widen(orc.narrow(ref, orc.F16), orc.F16), "matmul_t_f16", u16_dtype=orc.F16)


def test_matmul_transposed_whole_tiles(dev, stream, launcher):
    """256x512x768 f16 with B stored N x K over two logical tiles: the generated-assembly
    entry's transposed program."""
    tiles, M, K, N = 2, 256, 512, 768
    rng = np.random.default_rng(14)
    a = orc.narrow(rng.standard_normal(tiles * M * K).astype(np.float32), orc.F16)
    b = orc.narrow((rng.standard_normal(tiles * N * K) * 0.05).astype(np.float32), orc.F16)
    ab, bb = up(dev, stream, a, D.F16), up(dev, stream, b, D.F16)
    cb = dev.alloc(tiles * M * N, D.F16)
    launcher.launch("matmul_t_f16_tiles", th.LaunchGrid.blocks_only(tiles), [ptr(ab), ptr(bb), ptr(cb)],
                    stream)
    got = orc.widen(cb.copy_to_host(stream), orc.F16).reshape(tiles, M, N)
    for t in range(tiles):
        ref = orc.matmul(a[t * M * K:(t + 1) * M * K], b[t * N * K:(t + 1) * N * K], M, K, N,
                         orc.F16, orc.F32, b_trans=True)
        assert_gemm_close(got[t], orc.widen(orc.narrow(ref, orc.F16), orc.F16),
                          f"matmul_t_f16_tiles tile {t}", u16_dtype=orc.F16)


def test_matmul_f32_fma_integer_exact(dev, stream, launcher):
    M, K, N = 96, 72, 80
    rng = np.random.default_rng(5)
    a = rng.integers(-5, 6, (M, K)).astype(np.float32)
    b = rng.integers(-5, 6, (K, N)).astype(np.float32)
    ab, bb, cb = up(dev, stream, a, D.F32), up(dev, stream, b, D.F32), dev.alloc(M * N, D.F32)
    launcher.launch("matmul_f32", th.LaunchGrid.blocks_only(1), [ptr(ab), ptr(bb), ptr(cb)], stream)
    assert np.array_equal(cb.copy_to_host(stream).reshape(M, N), (a.astype(np.int64) @ b).astype(np.float32))


def test_rms_norm_rows_f32(dev, stream, launcher):
    tiles = 500  # 4 x 768 tiles
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((tiles * 4, 768)) * 1.5).astype(np.float32)
    xb, yb = up(dev, stream, x, D.F32), dev.alloc(x.size, D.F32)
    launcher.launch("rms_norm_rows_f32", th.LaunchGrid.blocks_only(tiles), [ptr(xb), ptr(yb)], stream)
    eps = float(np.float32(9.99999997e-7))
    assert_softmax_close(yb.copy_to_host(stream).reshape(tiles * 4, 768),
                         orc.rms_norm(x, tiles * 4, 768, eps), "emitted rms_norm")


def test_swiglu_gate_bf16_fused(dev, stream, launcher):
    tiles, M, K, N = 3, 256, 512, 256
    rng = np.random.default_rng(12)
    a = orc.narrow(rng.standard_normal(tiles * M * K).astype(np.float32), orc.BF16)
    b = orc.narrow((rng.standard_normal(tiles * K * N) * 0.05).astype(np.float32), orc.BF16)
    u = rng.standard_normal(tiles * M * N).astype(np.float32)
    ab, bb, ub = up(dev, stream, a, D.BF16), up(dev, stream, b, D.BF16), up(dev, stream, u, D.F32)
    cb = dev.alloc(tiles * M * N, D.F32)
    launcher.launch("swiglu_gate_bf16", th.LaunchGrid.blocks_only(tiles),
                    [ptr(ab), ptr(bb), ptr(ub), ptr(cb)], stream)
    got = cb.copy_to_host(stream).reshape(tiles, M, N)
    for t in range(tiles):
        ref = orc.matmul_silu_mul(a[t * M * K:(t + 1) * M * K], b[t * K * N:(t + 1) * K * N],
                                  u[t * M * N:(t + 1) * M * N], M, K, N, orc.BF16, orc.F32)
        assert_gemm_close(got[t], ref, f"emitted swiglu tile {t}")


def test_swiglu_gate_f16_whole_tiles(dev, stream, launcher):
    """256x512x512 f16 -> f16 over two logical tiles: the generated-assembly entry's
    SiLU*Mul program."""
    tiles, M, K, N = 2, 256, 512, 512
    rng = np.random.default_rng(15)
    a = orc.narrow(rng.standard_normal(tiles * M * K).astype(np.float32), orc.F16)
    b = orc.narrow((rng.standard_normal(tiles * K * N) * 0.05).astype(np.float32), orc.F16)
    u = orc.narrow(rng.standard_normal(tiles * M * N).astype(np.float32), orc.F16)
    ab, bb, ub = up(dev, stream, a, D.F16), up(dev, stream, b, D.F16), up(dev, stream, u, D.F16)
    cb = dev.alloc(tiles * M * N, D.F16)
    launcher.launch("swiglu_gate_f16", th.LaunchGrid.blocks_only(tiles),
                    [ptr(ab), ptr(bb), ptr(ub), ptr(cb)], stream)
    got = orc.widen(cb.copy_to_host(stream), orc.F16).reshape(tiles, M, N)
    for t in range(tiles):
        ref = orc.matmul_silu_mul(a[t * M * K:(t + 1) * M * K], b[t * K * N:(t + 1) * K * N],
                                  u[t * M * N:(t + 1) * M * N], M, K, N, orc.F16, orc.F16)
        assert_gemm_close(got[t], orc.widen(ref, orc.F16).reshape(M, N),
                          f"emitted swiglu f16 tile {t}", u16_dtype=orc.F16)


def test_attention_f32_tiles(dev, stream, launcher, golden):
    g = golden("attention_f32.npz")
    s, d = (int(t) for t in g["sd"])
    tiles = 2
    rng = np.random.default_rng(6)
    q = np.concatenate([g["q"].reshape(-1), rng.standard_normal(s * d).astype(np.float32)])
    k = np.concatenate([g["k"].reshape(-1), rng.standard_normal(s * d).astype(np.float32)])
    v = np.concatenate([g["v"].reshape(-1), rng.standard_normal(s * d).astype(np.float32)])
    bufs = [up(dev, stream, t, D.F32) for t in (q, k, v)]
    ob = dev.alloc(tiles * s * d, D.F32)
    launcher.launch("attention_f32", th.LaunchGrid.blocks_only(tiles), [ptr(b) for b in bufs] + [ptr(ob)],
                    stream)
    got = ob.copy_to_host(stream).reshape(tiles, s, d)
    assert np.abs(got[0] - g["o"]).max() < 1e-4
    ref1 = orc.attention_f32(q[s * d:], k[s * d:], v[s * d:], s, d)
    assert np.abs(got[1] - ref1).max() < 1e-5


@pytest.mark.parametrize("name,NH,NKV,S,Dh,dt", [("attention_gqa_f32", 8, 2, 32, 64, "f32"),
                                                   ("attention_gqa_wide_f32", 4, 1, 1500, 96, "f32"),
                                                   ("attention_gqa_bf16", 8, 2, 300, 128, "bf16")])
def test_attention_gqa_head_major(dev, stream, launcher, name, NH, NKV, S, Dh, dt):
    """__tile_attention_gqa_* (mlir_to_gpu.rs:1627-1712): causal GQA attention with
    Q/O [NH][S][D] and K/V [NKV][S][D], two logical tiles (batch elements); the
    oracle's token-major prefill on transposed Q/O is the reference."""
    B = 2
    rng = np.random.default_rng(NH * S + Dh)
    odt = orc.F32 if dt == "f32" else orc.BF16
    tdt = D.F32 if dt == "f32" else D.BF16
    def gen(n):
        x = rng.standard_normal(n).astype(np.float32)
        return x if dt == "f32" else orc.narrow(x, orc.BF16)
    q, k, v = gen(B * NH * S * Dh), gen(B * NKV * S * Dh), gen(B * NKV * S * Dh)
    bufs = [up(dev, stream, t, tdt) for t in (q, k, v)]
    ob = dev.alloc(q.size, tdt)
    launcher.launch(name, th.LaunchGrid.blocks_only(B), [ptr(b) for b in bufs] + [ptr(ob)], stream)
    got = ob.copy_to_host(stream)
    got = got if dt == "f32" else orc.widen(got, orc.BF16)
    q_tm = q.reshape(B, NH, S, Dh).transpose(0, 2, 1, 3).copy()
    ref = orc.attention_prefill(q_tm, k, v, odt, B, S, 0, S, Dh, NH, NKV)
    ref = ref.reshape(B, S, NH, Dh).transpose(0, 2, 1, 3).reshape(-1)
    if dt == "f32":
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
    else:
        assert_attn_close(got, ref, "head-major gqa")


@pytest.mark.parametrize("S,start,NH,NKV,Dh", [(200, 0, 4, 2, 128), (70, 9, 2, 1, 64), (600, 40, 8, 2, 64)])
def test_prefill_bf16(dev, stream, launcher, S, start, NH, NKV, Dh):
    B, max_seq = 2, start + S + 3
    rng = np.random.default_rng(S)
    q = orc.narrow(rng.standard_normal(B * S * NH * Dh).astype(np.float32), orc.BF16)
    k = orc.narrow(rng.standard_normal(B * NKV * max_seq * Dh).astype(np.float32), orc.BF16)
    v = orc.narrow(rng.standard_normal(B * NKV * max_seq * Dh).astype(np.float32), orc.BF16)
    bufs = [up(dev, stream, t, D.BF16) for t in (q, k, v)]
    ob = dev.alloc(q.size, D.BF16)
    scal = [C.c_uint32(x) for x in (S, start, max_seq, Dh, NH, NKV)]
    launcher.launch("prefill_bf16", th.LaunchGrid.blocks_only(B), [ptr(b) for b in bufs] + [ptr(ob)] + scal,
                    stream)
    got = orc.widen(ob.copy_to_host(stream), orc.BF16)
    ref = orc.attention_prefill(q, k, v, orc.BF16, B, S, start, max_seq, Dh, NH, NKV)
    assert_attn_close(got, ref, "emitted prefill")


@pytest.mark.parametrize("S,start,NH,NKV,Dh", [(300, 20, 8, 2, 128), (520, 64, 4, 4, 64)])
def test_prefill_bf16_same_bits_as_library(dev, stream, launcher, S, start, NH, NKV, Dh):
    """The emitted prefill runs the library's kernel with the same scale (its head-dim-128
    path folds 1/sqrt(128) at compile time): the two outputs match bit for bit."""
    B, max_seq = 2, start + S + 5
    rng = np.random.default_rng(S + Dh)
    q = orc.narrow(rng.standard_normal(B * S * NH * Dh).astype(np.float32), orc.BF16)
    k = orc.narrow(rng.standard_normal(B * NKV * max_seq * Dh).astype(np.float32), orc.BF16)
    v = orc.narrow(rng.standard_normal(B * NKV * max_seq * Dh).astype(np.float32), orc.BF16)
    bufs = [up(dev, stream, t, D.BF16) for t in (q, k, v)]
    oe, ol = dev.alloc(q.size, D.BF16), dev.alloc(q.size, D.BF16)
    scal = [C.c_uint32(x) for x in (S, start, max_seq, Dh, NH, NKV)]
    launcher.launch("prefill_bf16", th.LaunchGrid.blocks_only(B), [ptr(b) for b in bufs] + [ptr(oe)] + scal,
                    stream)
    th.attention_prefill(*bufs, ol, B, S, start, max_seq, Dh, NH, NKV, D.BF16, stream)
    np.testing.assert_array_equal(oe.copy_to_host(stream), ol.copy_to_host(stream))


@pytest.mark.parametrize("L,NH,NKV,Dh", [(700, 8, 2, 128), (1100, 16, 16, 128), (300, 6, 2, 128),
                                         (257, 4, 1, 64), (9000, 8, 2, 64), (600, 6, 2, 64)])
def test_decode_bf16(dev, stream, launcher, L, NH, NKV, Dh):
    B, max_seq = 3, L + 5
    rng = np.random.default_rng(L + NH)
    q = orc.narrow(rng.standard_normal(B * NH * Dh).astype(np.float32), orc.BF16)
    k = orc.narrow(rng.standard_normal(B * NKV * max_seq * Dh).astype(np.float32), orc.BF16)
    v = orc.narrow(rng.standard_normal(B * NKV * max_seq * Dh).astype(np.float32), orc.BF16)
    bufs = [up(dev, stream, t, D.BF16) for t in (q, k, v)]
    ob = dev.alloc(q.size, D.BF16)
    scal = [C.c_uint32(x) for x in (L, max_seq, Dh, NH, NKV)]
    launcher.launch("decode_bf16", th.LaunchGrid.blocks_only(B), [ptr(b) for b in bufs] + [ptr(ob)] + scal,
                    stream)
    got = orc.widen(ob.copy_to_host(stream), orc.BF16)
    ref = orc.attention_decode(q, k, v, orc.BF16, B, L, max_seq, Dh, NH, NKV)
    assert_attn_close(got, ref, "emitted decode")


def test_elementwise_swiglu_and_scaled_causal(dev, stream, launcher):
    rng = np.random.default_rng(7)
    tiles = 5
    gate = rng.standard_normal(tiles * 2 * 64).astype(np.float32)
    upv = rng.standard_normal(tiles * 2 * 64).astype(np.float32)
    gb, ub, ob = up(dev, stream, gate, D.F32), up(dev, stream, upv, D.F32), dev.alloc(gate.size, D.F32)
    launcher.launch("swiglu", th.LaunchGrid.blocks_only(tiles), [ptr(gb), ptr(ub), ptr(ob)], stream)
    g64 = gate.astype(np.float64)
    ref = g64 / (1 + np.exp(-g64)) * upv
    assert np.allclose(ob.copy_to_host(stream), ref, rtol=1e-5, atol=1e-6)

    x = (rng.standard_normal((3, 16, 16)) * 60).astype(np.float32)
    xb, yb = up(dev, stream, x, D.F32), dev.alloc(x.size, D.F32)
    launcher.launch("scaled_causal", th.LaunchGrid.blocks_only(3), [ptr(xb), ptr(yb)], stream)
    got = yb.copy_to_host(stream).reshape(3, 16, 16)
    want = np.clip(x * np.float32(0.125), -4, 4)
    for t in range(3):
        assert np.array_equal(got[t].view(np.uint32),
                              orc.causal_mask_f32(want[t], 16, 16).view(np.uint32))


def test_unknown_kernel_name_is_a_kernel_error(dev, stream, launcher):
    with pytest.raises(th.HalError) as e:
        launcher.launch("no_such_kernel", th.LaunchGrid.blocks_only(1), [], stream)
    assert e.value.kind == "KernelError" and "no_such_kernel" in str(e.value)


# ---- elementwise ops, row reductions, transpose and matvec (examples/ops_extra.mlir) ----

def _ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


@pytest.mark.parametrize("op,ulps", [("log", 2), ("tanh", 2), ("abs", 0), ("sqrt", 1),
                                     ("rsqrt", 2), ("sigmoid", 2), ("relu", 0)])
def test_elementwise_unary(dev, stream, launcher, op, ulps):
    tiles, n = 3, 4 * 256
    rng = np.random.default_rng(sum(map(ord, op)))
    x = (rng.standard_normal(tiles * n) * 3).astype(np.float32)
    if op in ("log", "sqrt", "rsqrt"):
        x = np.abs(x) + np.float32(1e-3)
    xb, yb = up(dev, stream, x, D.F32), dev.alloc(x.size, D.F32)
    launcher.launch(f"ew_{op}", th.LaunchGrid.blocks_only(tiles), [ptr(xb), ptr(yb)], stream)
    got = yb.copy_to_host(stream)
    d = _ulp_diff(got, orc.unary_f32(op, x))
    assert d.max() <= ulps, f"{op}: {d.max()} ulp"


def test_elementwise_min_and_four_operand_mul(dev, stream, launcher):
    tiles = 3
    rng = np.random.default_rng(31)
    a, b = (rng.standard_normal(tiles * 1024).astype(np.float32) for _ in range(2))
    ab, bb, yb = up(dev, stream, a, D.F32), up(dev, stream, b, D.F32), dev.alloc(a.size, D.F32)
    launcher.launch("ew_min", th.LaunchGrid.blocks_only(tiles), [ptr(ab), ptr(bb), ptr(yb)], stream)
    assert np.array_equal(yb.copy_to_host(stream), orc.minmax_f32("min", a, b))
    # mul(silu(g), u) with the four-operand binary form (a, b, rows, cols)
    g, u = (rng.standard_normal(2 * 1000).astype(np.float32) for _ in range(2))
    gb, ub, ob = up(dev, stream, g, D.F32), up(dev, stream, u, D.F32), dev.alloc(g.size, D.F32)
    launcher.launch("ew_silu_mul4", th.LaunchGrid.blocks_only(2), [ptr(gb), ptr(ub), ptr(ob)], stream)
    assert np.allclose(ob.copy_to_host(stream), orc.silu_mul(g, u), rtol=2e-6, atol=1e-7)


def test_nan_and_signed_zero_follow_maximumf_minimumf(dev, stream, launcher):
    """relu, max, min, clamp and the max / absmax row reductions lower as MLIR's
    arith.maximumf / arith.minimumf (mlir_to_linalg.rs:429, :788, :951-955, :1543): a
    NaN operand gives NaN and -0 orders below +0.  fmaxf / fminf would drop the NaN."""
    tiles, n = 2, 1024
    rng = np.random.default_rng(35)
    a, b = (rng.standard_normal(tiles * n).astype(np.float32) for _ in range(2))
    idx = np.arange(a.size)
    nan_a, nan_b = idx % 17 == 0, idx % 23 == 5
    z1 = (idx % 29 == 3) & ~nan_a & ~nan_b      # (-0, +0) pairs
    z2 = (idx % 31 == 4) & ~nan_a & ~nan_b & ~z1  # (+0, -0) pairs
    a[nan_a], b[nan_b] = np.nan, np.nan
    a[z1], b[z1] = -0.0, 0.0
    a[z2], b[z2] = 0.0, -0.0
    ab, bb, yb = up(dev, stream, a, D.F32), up(dev, stream, b, D.F32), dev.alloc(a.size, D.F32)

    def same_bits(got, ref, name):
        """NaN where the oracle has NaN; every other value bit-identical (signed zeros too)."""
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(got), nan), f"{name}: NaN positions differ"
        assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32)), name

    for op in ("min", "max"):
        launcher.launch(f"ew_{op}", th.LaunchGrid.blocks_only(tiles), [ptr(ab), ptr(bb), ptr(yb)], stream)
        same_bits(yb.copy_to_host(stream), orc.minmax_f32(op, a, b), op)
    launcher.launch("ew_relu", th.LaunchGrid.blocks_only(tiles), [ptr(ab), ptr(yb)], stream)
    got = yb.copy_to_host(stream)
    same_bits(got, orc.unary_f32("relu", a), "relu")
    assert np.isnan(got[nan_a]).all() and not np.signbit(got[z1]).any()
    launcher.launch("ew_clamp", th.LaunchGrid.blocks_only(tiles), [ptr(ab), ptr(yb)], stream)
    same_bits(yb.copy_to_host(stream), orc.clamp_f32(a, -0.5, 0.75), "clamp")
    R, C = 8, 1000
    x = rng.standard_normal(5 * R * C).astype(np.float32)
    x.reshape(-1, C)[2, 600] = np.nan
    x.reshape(-1, C)[11, 3] = np.nan
    xb, rb = up(dev, stream, x, D.F32), dev.alloc(5 * R, D.F32)
    for op in ("reduce_max", "absmax"):
        launcher.launch(f"row_{op}", th.LaunchGrid.blocks_only(5), [ptr(xb), ptr(rb)], stream)
        got = rb.copy_to_host(stream)
        ref = orc.reduce_rows_f32(op.replace("reduce_", ""), x, 5 * R, C)
        assert np.isnan(got[[2, 11]]).all() and np.isnan(ref[[2, 11]]).all(), op
        same_bits(got, ref, op)


@pytest.mark.parametrize("op", ["reduce_sum", "reduce_max", "absmax", "argmax"])
def test_row_reductions(dev, stream, launcher, op):
    tiles, R, C = 5, 8, 1000
    rng = np.random.default_rng(32)
    x = rng.standard_normal(tiles * R * C).astype(np.float32)
    xr = x.reshape(tiles * R, C)
    xr[3, 17] = xr[3, 900] = 9.0          # tied maxima: the first index wins
    xr[7, :] = -np.inf                      # nothing above -inf: index 0
    if op == "argmax":
        xr[7, 5] = -np.inf
    xb, yb = up(dev, stream, x, D.F32), dev.alloc(tiles * R, D.F32)
    launcher.launch(f"row_{op}", th.LaunchGrid.blocks_only(tiles), [ptr(xb), ptr(yb)], stream)
    got = yb.copy_to_host(stream)
    ref = orc.reduce_rows_f32(op.replace("reduce_", ""), x, tiles * R, C)
    if op == "argmax":
        assert np.array_equal(got.view(np.int32), ref)
        assert got.view(np.int32)[3] == 17 and got.view(np.int32)[7] == 0
    elif op == "reduce_sum":
        fin = np.isfinite(ref)
        bound = np.abs(xr[fin]).sum(axis=1) * 2e-7 + 1e-6
        assert (np.abs(got[fin] - ref[fin]) <= bound).all()
        assert np.array_equal(got[~fin], ref[~fin])
    else:
        assert np.array_equal(got, ref)


def test_row_sum_vectorised_rows(dev, stream, launcher):
    tiles, R, C = 4, 6, 4096
    rng = np.random.default_rng(33)
    xi = rng.integers(-64, 64, tiles * R * C).astype(np.float32)   # exact in any order
    xb, yb = up(dev, stream, xi, D.F32), dev.alloc(tiles * R, D.F32)
    launcher.launch("row_sum_aligned", th.LaunchGrid.blocks_only(tiles), [ptr(xb), ptr(yb)], stream)
    assert np.array_equal(yb.copy_to_host(stream), xi.reshape(-1, C).sum(axis=1))


def test_transpose_and_matvec(dev, stream, launcher):
    tiles = 3
    rng = np.random.default_rng(34)
    R, C = 48, 80
    x = rng.standard_normal(tiles * R * C).astype(np.float32)
    xb, yb = up(dev, stream, x, D.F32), dev.alloc(x.size, D.F32)
    launcher.launch("xpose", th.LaunchGrid.blocks_only(tiles), [ptr(xb), ptr(yb)], stream)
    got = yb.copy_to_host(stream).reshape(tiles, C * R)
    for t in range(tiles):
        assert np.array_equal(got[t], orc.transpose_f32(x[t * R * C:(t + 1) * R * C], R, C))
    R, C = 96, 200
    a = rng.standard_normal(tiles * R * C).astype(np.float32)
    v = rng.standard_normal(tiles * C).astype(np.float32)
    ab, vb, ob = up(dev, stream, a, D.F32), up(dev, stream, v, D.F32), dev.alloc(tiles * R, D.F32)
    launcher.launch("mv", th.LaunchGrid.blocks_only(tiles), [ptr(ab), ptr(vb), ptr(ob)], stream)
    got = ob.copy_to_host(stream).reshape(tiles, R)
    for t in range(tiles):
        at, vt = a[t * R * C:(t + 1) * R * C], v[t * C:(t + 1) * C]
        ref = orc.matvec_f32(at, vt, R, C)
        bound = np.abs(at.reshape(R, C)) @ np.abs(vt) * 2e-7 + 1e-6
        assert (np.abs(got[t] - ref) <= bound).all()


# ---- counted tile loops (tile.rs:2196-2210) -------------------------------------------------

def test_softmax_loop_runs_every_iteration(dev, stream, launcher):
    """The reference's loop example (a 1 x 1024 f32 softmax per iteration, n_tiles from the
    kernel argument, pipelined_for(2)): one launched tile walks all n rows; three
    launched tiles compute the same rows; n = 0 leaves the output untouched."""
    n = 300
    rng = np.random.default_rng(71)
    x = (rng.standard_normal((n, 1024)) * 2).astype(np.float32)
    ref = orc.softmax(x, n, 1024)
    xb = up(dev, stream, x, D.F32)
    for launched in (1, 3):
        yb = up(dev, stream, np.full(x.size + 1024, 7.0, np.float32), D.F32)
        launcher.launch("softmax_loop_f32", th.LaunchGrid.blocks_only(launched),
                        [ptr(xb), ptr(yb), C.c_uint32(n)], stream)
        got = yb.copy_to_host(stream)
        assert_softmax_close(got[:x.size].reshape(n, 1024), ref)
        assert np.all(got[x.size:] == 7.0), "the loop ran past n"
    yb = up(dev, stream, np.full(x.size, 7.0, np.float32), D.F32)
    launcher.launch("softmax_loop_f32", th.LaunchGrid.blocks_only(1),
                    [ptr(xb), ptr(yb), C.c_uint32(0)], stream)
    assert np.all(yb.copy_to_host(stream) == 7.0)


def test_softmax_loop_signed_bound(dev, stream, launcher):
    """`icmp slt %i, %n` with an i32 n: n = 300 walks 300 rows; a negative n runs no
    iteration (the kernel clamps its tile count and the grid stays one workgroup)."""
    n = 300
    rng = np.random.default_rng(74)
    x = (rng.standard_normal((n, 1024)) * 2).astype(np.float32)
    xb = up(dev, stream, x, D.F32)
    yb = up(dev, stream, np.full(x.size + 1024, 7.0, np.float32), D.F32)
    launcher.launch("softmax_loop_signed_f32", th.LaunchGrid.blocks_only(1),
                    [ptr(xb), ptr(yb), C.c_uint32(n)], stream)
    got = yb.copy_to_host(stream)
    assert_softmax_close(got[:x.size].reshape(n, 1024), orc.softmax(x, n, 1024))
    assert np.all(got[x.size:] == 7.0), "the loop ran past n"
    yb = up(dev, stream, np.full(x.size, 7.0, np.float32), D.F32)
    args = [ptr(xb), ptr(yb), C.c_int32(-5)]
    assert launcher.hardware_grid("softmax_loop_signed_f32", th.LaunchGrid.blocks_only(1), args)[0] == 1
    launcher.launch("softmax_loop_signed_f32", th.LaunchGrid.blocks_only(1), args, stream)
    assert np.all(yb.copy_to_host(stream) == 7.0)


def test_add_loop_i64_bound(dev, stream, launcher):
    """i64 trip count, `i < n` loop test, offsets from `i << 9` (2 x 256 tiles): exact."""
    n = 77
    rng = np.random.default_rng(72)
    a = rng.standard_normal(n * 512).astype(np.float32)
    b = rng.standard_normal(n * 512).astype(np.float32)
    ab, bb = up(dev, stream, a, D.F32), up(dev, stream, b, D.F32)
    cb = up(dev, stream, np.full(n * 512 + 512, 7.0, np.float32), D.F32)
    launcher.launch("add_loop_f32", th.LaunchGrid.blocks_only(1), [ptr(ab), ptr(bb), ptr(cb), C.c_uint64(n)],
                    stream)
    got = cb.copy_to_host(stream)
    np.testing.assert_array_equal(got[:n * 512], a + b)
    assert np.all(got[n * 512:] == 7.0)


def test_softmax_loop_generic_form_depth_one(dev, stream, launcher):
    """Generic-form loop, constant trip 48 over 4 x 512 bf16 tiles, pipelined_for(1)
    (the non-streaming row loop)."""
    rng = np.random.default_rng(73)
    rows = 48 * 4
    x = orc.narrow((rng.standard_normal(rows * 512) * 2).astype(np.float32), orc.BF16)
    xb, yb = up(dev, stream, x, D.BF16), dev.alloc(x.size, D.BF16)
    launcher.launch("softmax_loop_bf16_generic", th.LaunchGrid.blocks_only(1), [ptr(xb), ptr(yb)], stream)
    got = orc.widen(yb.copy_to_host(stream), orc.BF16)
    ref = orc.softmax(orc.widen(x, orc.BF16), rows, 512)
    assert_within_ulp16(got, ref.reshape(-1), orc.BF16)


def test_gemm_loop_is_a_batched_gemm(dev, stream, launcher):
    """A loop over n (A_i, B_i, C_i) views of 256x320x384 bf16 -> f32 GEMMs with
    pipelined_for(5) (a 5-stage LDS ring): n batch entries of the DMA GEMM."""
    n, M, K, N = 3, 256, 320, 384
    rng = np.random.default_rng(74)
    a = orc.narrow(rng.uniform(-1, 1, n * M * K).astype(np.float32), orc.BF16)
    b = orc.narrow(rng.uniform(-1, 1, n * K * N).astype(np.float32), orc.BF16)
    ab, bb = up(dev, stream, a, D.BF16), up(dev, stream, b, D.BF16)
    cb = up(dev, stream, np.full(n * M * N + 64, 7.0, np.float32), D.F32)
    launcher.launch("gemm_loop_bf16", th.LaunchGrid.blocks_only(1), [ptr(ab), ptr(bb), ptr(cb), C.c_uint32(n)],
                    stream)
    got = cb.copy_to_host(stream)
    assert np.all(got[n * M * N:] == 7.0)
    for i in range(n):
        ref = orc.matmul(a[i * M * K:(i + 1) * M * K], b[i * K * N:(i + 1) * K * N], M, K, N, orc.BF16)
        assert_gemm_close(got[i * M * N:(i + 1) * M * N].reshape(M, N), ref.reshape(M, N), f"loop GEMM {i}")

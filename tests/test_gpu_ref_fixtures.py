"""The reference's own hot-path MLIR test inputs, run on the GPU against the oracle.

Each module below is one of the reference's test constants, stored verbatim as data
under tests/golden/ref_mlir (tests/golden/extract_ref_mlir.py):

  linalg__matmul                  MATMUL                   mlir_to_linalg.rs:1941
  linalg__softmax                 SOFTMAX                  mlir_to_linalg.rs:1957
  linalg__attention               ATTENTION                mlir_to_linalg.rs:2088
  linalg__attention_decode_kernel ATTENTION_DECODE_KERNEL  mlir_to_linalg.rs:2550
  linalg__rms_norm                RMS_NORM                 mlir_to_linalg.rs:2629
  linalg__attn_prefill_mlir       ATTN_PREFILL_MLIR        mlir_to_linalg.rs:2978
  gpu__softmax_mlir_0             softmax test             mlir_to_gpu.rs:2185
  gpu__matmul_f16_mlir_0          matmul_f16 test          mlir_to_gpu.rs:2612
  gpu__attention_gqa_mlir_0       attention_gqa test       mlir_to_gpu.rs:2995

The build emits each through the `hip` target and compiles it for gfx950
(tilers_hip/_build.py REF_HOT_PATH); these tests launch the code objects through
th_launcher_launch at the modules' own tile shapes, several logical tiles per launch
(the #[tile_kernel] per-tile offsets), and compare every output element with the
oracle.  The decode and prefill kernels take their runtime sizes as trailing scalars
in the Metal target's order (mlir_to_msl.rs:1816-1823, :1851-1859).

Tolerances: f32 softmax and RMSNorm 1e-5 relative; f32 GEMM the GEMM bound of
tests/tolerances.py; f32 attention 1e-5 absolute on outputs of size ~1 (weighted
means of V ~ N(0, 1)); the f16 GEMM the GEMM bound plus one f16 ulp.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import tilers_hip as th
from oracle import oracle as orc
from tests.tolerances import assert_gemm_close, assert_softmax_close
from tilers_hip import _build

pytestmark = pytest.mark.gpu
D = th.TileDtype
F32_ATTN_ATOL = 1e-5


def load(dev, stem):
    lau = dev.create_launcher()
    lau.load(_build.ref_fixture_path(stem), th.KernelMode.GENERAL)
    return lau


def up(dev, s, a, dt):
    b = dev.alloc(a.size, dt)
    b.copy_from_host(np.ascontiguousarray(a).reshape(-1), s)
    return b


def ptr(b):
    return C.c_void_p(b.as_raw_ptr())


def u32(*xs):
    return [C.c_uint32(x) for x in xs]


def assert_attn_f32(got, ref, name):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    assert err.max() < F32_ATTN_ATOL, f"{name}: max err {err.max():.3e} at {np.argmax(err)}"


def test_all_hot_path_fixtures_are_built():
    for stem in _build.REF_HOT_PATH:
        assert _build.ref_fixture_path(stem).exists(), stem


def test_linalg_matmul(dev, stream):
    """MATMUL: __tile_matmul_f32 128x128x128 -> the fp32 MFMA GEMM, three tiles."""
    lau = load(dev, "linalg__matmul")
    T, M = 3, 128
    rng = np.random.default_rng(1941)
    a = rng.standard_normal(T * M * M).astype(np.float32)
    b = (rng.standard_normal(T * M * M) * 0.1).astype(np.float32)
    ab, bb, cb = up(dev, stream, a, D.F32), up(dev, stream, b, D.F32), dev.alloc(T * M * M, D.F32)
    lau.launch("tile_matmul", th.LaunchGrid.blocks_only(T), [ptr(ab), ptr(bb), ptr(cb)], stream)
    got = cb.copy_to_host(stream).reshape(T, M, M)
    for t in range(T):
        sl = slice(t * M * M, (t + 1) * M * M)
        ref = orc.matmul(a[sl], b[sl], M, M, M, orc.F32)
        assert_gemm_close(got[t], ref, f"MATMUL tile {t}")
    # integer-valued operands: every partial sum is exact, so the result is too
    ai = rng.integers(-8, 9, T * M * M).astype(np.float32)
    bi = rng.integers(-8, 9, T * M * M).astype(np.float32)
    ab.copy_from_host(ai, stream)
    bb.copy_from_host(bi, stream)
    lau.launch("tile_matmul", th.LaunchGrid.blocks_only(T), [ptr(ab), ptr(bb), ptr(cb)], stream)
    got = cb.copy_to_host(stream).reshape(T, M, M)
    for t in range(T):
        ref = ai[t * M * M:(t + 1) * M * M].reshape(M, M).astype(np.int64) @ \
            bi[t * M * M:(t + 1) * M * M].reshape(M, M).astype(np.int64)
        assert np.array_equal(got[t], ref.astype(np.float32)), f"MATMUL integer tile {t}"


@pytest.mark.parametrize("stem", ["linalg__softmax", "gpu__softmax_mlir_0"])
def test_softmax_fixtures(dev, stream, stem):
    """SOFTMAX and the gpu emitter's softmax test: 1 x 1024 f32 rows, 777 tiles."""
    lau = load(dev, stem)
    T, cols = 777, 1024
    rng = np.random.default_rng(1957)
    x = (rng.standard_normal((T, cols)) * 2.0).astype(np.float32)
    x[5] = 3.0                              # a constant row: every output 1/1024
    x[9, 17] = 80.0                         # one dominant entry
    xb, yb = up(dev, stream, x, D.F32), dev.alloc(x.size, D.F32)
    lau.launch("tile_softmax", th.LaunchGrid.cuda(T, cols), [ptr(xb), ptr(yb)], stream)
    y = yb.copy_to_host(stream).reshape(T, cols)
    assert_softmax_close(y, orc.softmax(x, T, cols), stem)
    assert np.all(y[5] == np.float32(1.0 / 1024))


def test_linalg_rms_norm(dev, stream):
    """RMS_NORM: 1 x 256 f32 rows, eps 1e-5, 1000 tiles."""
    lau = load(dev, "linalg__rms_norm")
    T, cols = 1000, 256
    rng = np.random.default_rng(2629)
    x = (rng.standard_normal((T, cols)) * 1.5).astype(np.float32)
    xb, yb = up(dev, stream, x, D.F32), dev.alloc(x.size, D.F32)
    lau.launch("tile_rms", th.LaunchGrid.blocks_only(T), [ptr(xb), ptr(yb)], stream)
    eps = float(np.float32(1.0e-5))
    assert_softmax_close(yb.copy_to_host(stream).reshape(T, cols), orc.rms_norm(x, T, cols, eps),
                         "RMS_NORM")


def test_linalg_attention(dev, stream):
    """ATTENTION: single-head f32 attention S=128 D=64 (the fp32 MFMA flash kernel),
    two tiles."""
    lau = load(dev, "linalg__attention")
    T, S, Dh = 2, 128, 64
    rng = np.random.default_rng(2088)
    q, k, v = (rng.standard_normal(T * S * Dh).astype(np.float32) for _ in range(3))
    bufs = [up(dev, stream, t, D.F32) for t in (q, k, v)]
    ob = dev.alloc(T * S * Dh, D.F32)
    lau.launch("tile_attention", th.LaunchGrid.blocks_only(T), [ptr(b) for b in bufs] + [ptr(ob)],
               stream)
    got = ob.copy_to_host(stream).reshape(T, S, Dh)
    for t in range(T):
        sl = slice(t * S * Dh, (t + 1) * S * Dh)
        assert_attn_f32(got[t], orc.attention_f32(q[sl], k[sl], v[sl], S, Dh), f"ATTENTION tile {t}")


@pytest.mark.parametrize("B,L,max_seq,Dh,NH,NKV", [(2, 700, 710, 128, 8, 2), (3, 1, 4, 64, 4, 4),
                                                   (1, 2000, 2000, 128, 16, 1)])
def test_linalg_attention_decode(dev, stream, B, L, max_seq, Dh, NH, NKV):
    """ATTENTION_DECODE_KERNEL (f32), runtime (seq_len, max_seq, head_dim, num_heads,
    num_kv_heads); B logical tiles = batch elements."""
    lau = load(dev, "linalg__attention_decode_kernel")
    rng = np.random.default_rng(2550 + L)
    q = rng.standard_normal(B * NH * Dh).astype(np.float32)
    k, v = (rng.standard_normal(B * NKV * max_seq * Dh).astype(np.float32) for _ in range(2))
    bufs = [up(dev, stream, t, D.F32) for t in (q, k, v)]
    ob = dev.alloc(B * NH * Dh, D.F32)
    lau.launch("tile_attn_decode", th.LaunchGrid.blocks_only(B),
               [ptr(b) for b in bufs] + [ptr(ob)] + u32(L, max_seq, Dh, NH, NKV), stream)
    ref = orc.attention_decode(q, k, v, orc.F32, B, L, max_seq, Dh, NH, NKV)
    assert_attn_f32(ob.copy_to_host(stream), ref, f"ATTENTION_DECODE_KERNEL B{B} L{L}")


@pytest.mark.parametrize("B,S,start,extra,Dh,NH,NKV", [(2, 100, 37, 13, 64, 4, 2),
                                                       (1, 300, 0, 0, 128, 8, 8),
                                                       (1, 4, 0, 0, 64, 1, 1)])
def test_linalg_attn_prefill(dev, stream, B, S, start, extra, Dh, NH, NKV):
    """ATTN_PREFILL_MLIR (f32), runtime (seq_len, start_pos, max_seq, head_dim,
    num_heads, num_kv_heads); the last case is the module's own 4 x 64 tile as one head."""
    lau = load(dev, "linalg__attn_prefill_mlir")
    max_seq = start + S + extra
    rng = np.random.default_rng(2978 + S)
    q = rng.standard_normal(B * S * NH * Dh).astype(np.float32)
    k, v = (rng.standard_normal(B * NKV * max_seq * Dh).astype(np.float32) for _ in range(2))
    bufs = [up(dev, stream, t, D.F32) for t in (q, k, v)]
    ob = dev.alloc(q.size, D.F32)
    lau.launch("ak", th.LaunchGrid.blocks_only(B),
               [ptr(b) for b in bufs] + [ptr(ob)] + u32(S, start, max_seq, Dh, NH, NKV), stream)
    ref = orc.attention_prefill(q, k, v, orc.F32, B, S, start, max_seq, Dh, NH, NKV)
    assert_attn_f32(ob.copy_to_host(stream), ref, f"ATTN_PREFILL_MLIR B{B} S{S} start{start}")


def test_gpu_matmul_f16(dev, stream):
    """The gpu emitter's matmul_f16 test: 32x64 . 64x32 f16 -> f16, four tiles."""
    lau = load(dev, "gpu__matmul_f16_mlir_0")
    T, M, K, N = 4, 32, 64, 32
    rng = np.random.default_rng(2612)
    a = orc.narrow(rng.standard_normal(T * M * K).astype(np.float32), orc.F16)
    b = orc.narrow((rng.standard_normal(T * K * N) * 0.2).astype(np.float32), orc.F16)
    ab, bb, cb = up(dev, stream, a, D.F16), up(dev, stream, b, D.F16), dev.alloc(T * M * N, D.F16)
    lau.launch("tile_matmul_f16", th.LaunchGrid.blocks_only(T), [ptr(ab), ptr(bb), ptr(cb)], stream)
    got = orc.widen(cb.copy_to_host(stream), orc.F16).reshape(T, M, N)
    for t in range(T):
        ref = orc.matmul(a[t * M * K:(t + 1) * M * K], b[t * K * N:(t + 1) * K * N], M, K, N,
                         orc.F16, orc.F32)
        assert_gemm_close(got[t], orc.widen(orc.narrow(ref, orc.F16), orc.F16).reshape(M, N),
                          f"matmul_f16 tile {t}", u16_dtype=orc.F16)


def test_gpu_attention_gqa(dev, stream):
    """The gpu emitter's attention_gqa test: causal GQA, head-major Q/O [8][32][64],
    K/V [2][32][64] f32, two tiles; the oracle's token-major prefill on transposed Q/O."""
    lau = load(dev, "gpu__attention_gqa_mlir_0")
    B, NH, NKV, S, Dh = 2, 8, 2, 32, 64
    rng = np.random.default_rng(2995)
    q = rng.standard_normal(B * NH * S * Dh).astype(np.float32)
    k, v = (rng.standard_normal(B * NKV * S * Dh).astype(np.float32) for _ in range(2))
    bufs = [up(dev, stream, t, D.F32) for t in (q, k, v)]
    ob = dev.alloc(q.size, D.F32)
    lau.launch("tile_attention_gqa", th.LaunchGrid.blocks_only(B), [ptr(b) for b in bufs] + [ptr(ob)],
               stream)
    q_tm = q.reshape(B, NH, S, Dh).transpose(0, 2, 1, 3).copy()
    ref = orc.attention_prefill(q_tm, k, v, orc.F32, B, S, 0, S, Dh, NH, NKV)
    ref = ref.reshape(B, S, NH, Dh).transpose(0, 2, 1, 3).reshape(-1)
    assert_attn_f32(ob.copy_to_host(stream), ref, "attention_gqa")

"""GPU parity: every tile op through the C ABI vs the CPU oracle (MI355X only).

Inputs are seeded; the HIP result and the oracle see identical bytes.  Full
BASELINE sizes are checked on every output element (config 4 through the
session-wide oracle result of tests/conftest.py), small and ragged shapes in
full.  Tolerances: tests/tolerances.py.
"""
from __future__ import annotations

import numpy as np
import pytest

import tilers_hip as th
from oracle import oracle as orc
from tests.tolerances import (assert_attn_close, assert_gemm_close, assert_softmax_close,
                              assert_within_ulp16)

pytestmark = pytest.mark.gpu

D = th.TileDtype
ORC = {D.F32: orc.F32, D.F16: orc.F16, D.BF16: orc.BF16}


def upload(dev, stream, arr: np.ndarray, dtype: th.TileDtype) -> th.HipBuffer:
    buf = dev.alloc(arr.size, dtype)
    buf.copy_from_host(np.ascontiguousarray(arr).reshape(-1), stream)
    return buf


def rand16(rng, n, dtype, scale=1.0, kind="normal"):
    x = rng.standard_normal(n) if kind == "normal" else rng.uniform(-1, 1, n)
    return orc.narrow((x * scale).astype(np.float32), ORC[dtype])


def device_random(dev, stream, n, dtype, dist, p0, p1, seed):
    buf = dev.alloc(n, dtype)
    th.fill_random(buf, n, dtype, dist, p0, p1, seed, stream)
    return buf


# ---- device / runtime -------------------------------------------------------------

def test_device_properties(dev):
    assert dev.arch().startswith("gfx950")
    assert dev.cu_count() > 0
    mi = dev.mem_info()
    assert mi.total > 100 * 2 ** 30 and 0 < mi.free <= mi.total
    print(f"device {dev.name()} {dev.arch()} cus={dev.cu_count()} mem={mi.total / 2**30:.0f} GiB")


def test_buffer_round_trip(dev, stream):
    x = np.arange(1000, dtype=np.float32)
    b = dev.alloc_from_slice(x, stream)
    assert len(b) == 1000
    assert np.array_equal(b.copy_to_host(stream), x)


def test_fill_random_moments(dev, stream):
    n = 1 << 20
    b = device_random(dev, stream, n, D.F32, "normal", 0.0, 2.0, 0x71130001)
    x = b.copy_to_host(stream)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 2.0) < 0.01
    u = device_random(dev, stream, n, D.BF16, "uniform", -1.0, 1.0, 0x71130002).copy_to_host(stream)
    uf = orc.widen(u, orc.BF16)
    assert uf.min() >= -1.0 and uf.max() <= 1.0 and abs(uf.mean()) < 0.01
    again = device_random(dev, stream, n, D.F32, "normal", 0.0, 2.0, 0x71130001).copy_to_host(stream)
    assert np.array_equal(again, x)  # counter-based: same seed, same bytes


def test_errors_are_hal_errors(dev, stream):
    with pytest.raises(th.HalError) as e:
        th.attention_prefill(1, 1, 1, 1, 1, 8, 0, 4, 128, 4, 4, D.BF16, stream)
    assert e.value.kind == "KernelError" and "max_seq" in str(e.value)
    with pytest.raises(th.HalError) as e:
        th.attention_decode(1, 1, 1, 1, 1, 8, 8, 128, 6, 4, D.BF16, stream=stream)
    assert e.value.kind == "KernelError"


def test_empty_and_degenerate_sizes(dev, stream):
    """Zero rows / M / batch / seq_len launch nothing and leave the output untouched;
    an empty contraction (K = 0) writes C = 0 (linalg.fill 0 with nothing accumulated,
    mlir_to_linalg.rs:1345-1393); a decode over zero positions writes O = 0."""
    sentinel = np.full(256, 7.0, np.float32)
    x = upload(dev, stream, sentinel, D.F32)
    y = upload(dev, stream, sentinel, D.F32)
    th.softmax(x, y, 0, 256, D.F32, stream)
    th.rms_norm(x, y, 0, 256, 1e-6, D.F32, stream)
    th.matmul(x, x, y, 0, 16, 16, D.F32, D.F32, stream=stream)
    th.matmul(x, x, y, 16, 16, 16, D.F32, D.F32, batch=0, stream=stream)
    assert np.array_equal(y.copy_to_host(stream), sentinel)
    th.matmul(x, x, y, 8, 0, 16, D.F32, D.F32, stream=stream)
    out = y.copy_to_host(stream)
    assert np.all(out[:128] == 0.0) and np.array_equal(out[128:], sentinel[128:])
    q16 = upload(dev, stream, orc.narrow(sentinel, orc.BF16), D.BF16)
    o16 = upload(dev, stream, orc.narrow(sentinel, orc.BF16), D.BF16)
    th.attention_prefill(q16, q16, q16, o16, 1, 0, 0, 4, 128, 2, 2, D.BF16, stream)
    assert np.array_equal(o16.copy_to_host(stream), orc.narrow(sentinel, orc.BF16))
    th.attention_decode(q16, q16, q16, o16, 1, 0, 4, 128, 2, 2, D.BF16, stream=stream)
    assert np.all(o16.copy_to_host(stream) == 0)


# ---- softmax ------------------------------------------------------------------------

def test_softmax_golden_vectors(dev, stream, golden):
    g = golden("softmax_f32.npz")
    x = g["x"]
    xb = upload(dev, stream, x, D.F32)
    yb = dev.alloc(x.size, D.F32)
    th.softmax(xb, yb, *x.shape, D.F32, stream)
    y = yb.copy_to_host(stream).reshape(x.shape)
    assert_softmax_close(y, g["y"], "softmax golden")


def test_softmax_config1_full(dev, stream):
    """8192 x 1024 f32, X ~ N(0, 2.0), full tensor, rel 1e-5."""
    rows, cols = 8192, 1024
    xb = device_random(dev, stream, rows * cols, D.F32, "normal", 0.0, 2.0, 0x71130000 + 1)
    yb = dev.alloc(rows * cols, D.F32)
    th.softmax(xb, yb, rows, cols, D.F32, stream)
    x = xb.copy_to_host(stream).reshape(rows, cols)
    y = yb.copy_to_host(stream).reshape(rows, cols)
    ref = orc.softmax(x, rows, cols)
    assert_softmax_close(y, ref, "softmax config1")
    assert np.allclose(y.astype(np.float64).sum(axis=1), 1.0, atol=1e-5)


@pytest.mark.parametrize("rows,cols", [(3, 1000), (5, 77), (7, 1), (2, 5000), (33, 4096),
                                       (4, 256), (1, 64), (9, 17000),
                                       # many rows per wave in the streaming kernel, ragged tail
                                       (12345, 256), (20001, 128), (9000, 1024), (5000, 60),
                                       # rows of 513-1024 16-byte vectors, >= CU-count rows:
                                       # the streaming workgroup form (ragged last vector)
                                       (300, 4096), (1000, 2056)])
def test_softmax_f32_shapes(dev, stream, rows, cols):
    rng = np.random.default_rng(rows * 131 + cols)
    x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
    xb = upload(dev, stream, x, D.F32)
    yb = dev.alloc(x.size, D.F32)
    th.softmax(xb, yb, rows, cols, D.F32, stream)
    assert_softmax_close(yb.copy_to_host(stream).reshape(rows, cols), orc.softmax(x, rows, cols),
                         f"softmax {rows}x{cols}")


@pytest.mark.parametrize("dtype", [D.F16, D.BF16])
@pytest.mark.parametrize("rows,cols", [(64, 2048), (3, 100), (4, 8192), (17003, 512),
                                       (512, 8192), (300, 5000)])
def test_softmax_u16(dev, stream, dtype, rows, cols):
    rng = np.random.default_rng(cols)
    x = rand16(rng, rows * cols, dtype, 2.0)
    xb = upload(dev, stream, x, dtype)
    yb = dev.alloc(x.size, dtype)
    th.softmax(xb, yb, rows, cols, dtype, stream)
    y = orc.widen(yb.copy_to_host(stream), ORC[dtype])
    ref = orc.softmax(orc.widen(x, ORC[dtype]), rows, cols)
    assert_within_ulp16(y, ref, ORC[dtype], 1.0, f"softmax {dtype.name} {rows}x{cols}")


@pytest.mark.parametrize("rows,cols", [(1, 1 << 20), (64, 131072), (3, 100003), (256, 32000),
                                       (1, 2049), (2, 8 * 4096 + 4),
                                       # enough rows for one workgroup per row in registers
                                       (300, 8000), (512, 16384), (300, 8001)])
def test_softmax_long_rows_f32(dev, stream, rows, cols):
    """Rows split over several workgroups (chunk statistics merged per row), or one
    workgroup per row when the rows fill the chip; ragged and unaligned column counts
    take the scalar form of the split kernels."""
    rng = np.random.default_rng(rows * 7 + cols)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    xb = upload(dev, stream, x, D.F32)
    yb = dev.alloc(x.size, D.F32)
    th.softmax(xb, yb, rows, cols, D.F32, stream)
    y = yb.copy_to_host(stream).reshape(rows, cols)
    assert_softmax_close(y, orc.softmax(x, rows, cols), f"softmax {rows}x{cols}")
    assert np.allclose(y.astype(np.float64).sum(axis=1), 1.0, atol=1e-5)


@pytest.mark.parametrize("dtype", [D.F16, D.BF16])
@pytest.mark.parametrize("rows,cols", [(3, 152064), (2048, 32000), (5, 70001)])
def test_softmax_long_rows_u16(dev, stream, dtype, rows, cols):
    rng = np.random.default_rng(cols + rows)
    x = rand16(rng, rows * cols, dtype, 2.0)
    xb = upload(dev, stream, x, dtype)
    yb = dev.alloc(x.size, dtype)
    th.softmax(xb, yb, rows, cols, dtype, stream)
    y = orc.widen(yb.copy_to_host(stream), ORC[dtype])
    ref = orc.softmax(orc.widen(x, ORC[dtype]), rows, cols)
    assert_within_ulp16(y, ref, ORC[dtype], 1.0, f"softmax {dtype.name} {rows}x{cols}")


def test_softmax_long_rows_masked_and_in_place(dev, stream):
    """A long row whose first 60000 entries are -inf (whole chunks with no finite value)
    next to an unmasked row; computed in place."""
    rows, cols = 2, 200000
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
    x[0, :60000] = -np.inf
    x[1, 199990:] = -np.inf
    b = upload(dev, stream, x, D.F32)
    th.softmax(b, b, rows, cols, D.F32, stream)
    y = b.copy_to_host(stream).reshape(rows, cols)
    ref = orc.softmax(x, rows, cols)
    assert np.all(y[0, :60000] == 0.0) and np.all(y[1, 199990:] == 0.0)
    assert_softmax_close(y, ref, "softmax masked long rows")


@pytest.mark.parametrize("x_off,y_off", [(1, 1), (1, 2), (0, 3)])
def test_row_ops_offset_pointers(dev, stream, x_off, y_off):
    """Long ragged rows at element offsets: the same 16-byte phase for x and y (vector
    middle between scalar head and tail) and different phases (scalar apply)."""
    rows, cols = 4, 50257
    rng = np.random.default_rng(x_off * 10 + y_off)
    x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
    xb = upload(dev, stream, np.concatenate([np.zeros(x_off, np.float32), x.reshape(-1)]), D.F32)
    yb = dev.alloc(rows * cols + y_off, D.F32)
    xp, yp = xb.as_raw_ptr() + 4 * x_off, yb.as_raw_ptr() + 4 * y_off
    th.softmax(xp, yp, rows, cols, D.F32, stream)
    y = yb.copy_to_host(stream)[y_off:].reshape(rows, cols)
    assert_softmax_close(y, orc.softmax(x, rows, cols), "softmax offset pointers")
    th.rms_norm(xp, yp, rows, cols, 1e-6, D.F32, stream)
    y = yb.copy_to_host(stream)[y_off:].reshape(rows, cols)
    assert_softmax_close(y, orc.rms_norm(x, rows, cols, 1e-6), "rms_norm offset pointers")


def test_softmax_in_place(dev, stream):
    rng = np.random.default_rng(99)
    x = rng.standard_normal((16, 1024)).astype(np.float32)
    b = upload(dev, stream, x, D.F32)
    th.softmax(b, b, 16, 1024, D.F32, stream)
    assert_softmax_close(b.copy_to_host(stream).reshape(16, 1024), orc.softmax(x, 16, 1024))


# ---- matmul -------------------------------------------------------------------------

def test_matmul_golden_vectors(dev, stream, golden):
    for name, dt, trans in (("matmul_bf16.npz", D.BF16, False), ("matmul_f16_t.npz", D.F16, True)):
        g = golden(name)
        m, k, n = (int(t) for t in g["mkn"])
        a = upload(dev, stream, g["a"], dt)
        b = upload(dev, stream, g["b"], dt)
        c = dev.alloc(m * n, D.F32)
        th.matmul(a, b, c, m, k, n, dt, D.F32, trans, stream=stream)
        assert_gemm_close(c.copy_to_host(stream).reshape(m, n), g["c"], name)


@pytest.mark.parametrize("in_dt", [D.BF16, D.F16, D.F32])
@pytest.mark.parametrize("trans", [False, True])
@pytest.mark.parametrize("m,k,n", [(256, 256, 256), (300, 72, 136), (1, 8, 8), (513, 1024, 264),
                                   (64, 33, 40), (512, 96, 768), (768, 1024, 512), (1, 64, 8),
                                   (40, 64, 36), (40, 32, 36), (300, 160, 264)])
def test_matmul_integer_bit_exact(dev, stream, in_dt, trans, m, k, n):
    """Integer-valued inputs make every partial sum exact: any layout/index slip shows."""
    rng = np.random.default_rng(m + 7 * k + 13 * n)
    a = rng.integers(-4, 5, (m, k)).astype(np.float32)
    b = rng.integers(-4, 5, (n, k) if trans else (k, n)).astype(np.float32)
    ref = (a.astype(np.int64) @ (b.T if trans else b).astype(np.int64)).astype(np.float32)
    ab = upload(dev, stream, orc.narrow(a, ORC[in_dt]), in_dt)
    bb = upload(dev, stream, orc.narrow(b, ORC[in_dt]), in_dt)
    cb = dev.alloc(m * n, D.F32)
    th.matmul(ab, bb, cb, m, k, n, in_dt, D.F32, trans, stream=stream)
    got = cb.copy_to_host(stream).reshape(m, n)
    assert np.array_equal(got, ref), f"max diff {np.abs(got - ref).max()}"


@pytest.mark.parametrize("trans", [False, True])
@pytest.mark.parametrize("in_dt", [D.BF16, D.F16])
@pytest.mark.parametrize("out_dt", [D.F32, D.BF16, D.F16])
@pytest.mark.parametrize("m,k,n,bsz", [(256, 256, 256, 1), (512, 384, 768, 1), (768, 1152, 512, 1),
                                       (256, 512, 512, 3)])
def test_matmul_whole_tiles_bit_exact(dev, stream, trans, in_dt, out_dt, m, k, n, bsz):
    """Whole 256 x 256 tiles, K a multiple of 128, B row-major or stored N x K: the
    generated-assembly kernel (K in 8, 12 and 36 steps of 32, and a batch).  Integer
    inputs keep every f32 partial sum exact, so C is the exact product rounded once to
    its dtype."""
    rng = np.random.default_rng(m + 3 * k + 5 * n + bsz)
    a = rng.integers(-4, 5, (bsz, m, k)).astype(np.float32)
    b = rng.integers(-4, 5, (bsz, k, n)).astype(np.float32)
    bs = np.ascontiguousarray(b.transpose(0, 2, 1)) if trans else b
    ab = upload(dev, stream, orc.narrow(a.ravel(), ORC[in_dt]), in_dt)
    bb = upload(dev, stream, orc.narrow(bs.ravel(), ORC[in_dt]), in_dt)
    cb = dev.alloc(bsz * m * n, out_dt)
    th.matmul(ab, bb, cb, m, k, n, in_dt, out_dt, trans, batch=bsz, stream=stream)
    raw = cb.copy_to_host(stream).reshape(bsz, m, n)
    for i in range(bsz):
        ref = (a[i].astype(np.int64) @ b[i].astype(np.int64)).astype(np.float32)
        if out_dt == D.F32:
            assert np.array_equal(raw[i], ref), f"batch {i}: max diff {np.abs(raw[i] - ref).max()}"
        else:
            want = orc.narrow(ref.ravel(), ORC[out_dt]).reshape(m, n)
            assert np.array_equal(raw[i], want), f"batch {i}: {np.sum(raw[i] != want)} elements differ"


@pytest.mark.parametrize("m,k,n,trans,out_dt,bsz", [
    (1000, 777, 1030, False, D.F32, 1),    # ragged in every dimension, K % 4 != 0
    (513, 1024, 264, True, D.F32, 2),      # B stored N x K, batched
    (256, 4096, 384, False, D.F16, 1),     # long K, 16-bit output
    (130, 20, 5, True, D.BF16, 3),         # one partial tile per batch entry
])
def test_matmul_f32_mfma(dev, stream, m, k, n, trans, out_dt, bsz):
    """f32 operands on the fp32 MFMA kernel against the oracle's sequential f32 FMA;
    the K sum runs in another order, so the check is the GEMM tolerance."""
    rng = np.random.default_rng(m * 3 + k + n + bsz)
    a = rng.standard_normal(bsz * m * k).astype(np.float32)
    b = (rng.standard_normal(bsz * k * n) * 0.05).astype(np.float32)
    ab, bb = upload(dev, stream, a, D.F32), upload(dev, stream, b, D.F32)
    cb = dev.alloc(bsz * m * n, out_dt)
    th.matmul(ab, bb, cb, m, k, n, D.F32, out_dt, trans, batch=bsz, stream=stream)
    raw = cb.copy_to_host(stream)
    got = (raw if out_dt == D.F32 else orc.widen(raw, ORC[out_dt])).reshape(bsz, m, n)
    for i in range(bsz):
        ref = orc.matmul(a[i * m * k:(i + 1) * m * k], b[i * k * n:(i + 1) * k * n], m, k, n,
                         orc.F32, ORC[out_dt], b_trans=trans)
        ref32 = ref if out_dt == D.F32 else orc.widen(ref, ORC[out_dt])
        assert_gemm_close(got[i], ref32.reshape(m, n), f"f32 {m}x{k}x{n} batch {i}",
                          u16_dtype=None if out_dt == D.F32 else ORC[out_dt])


@pytest.mark.parametrize("out_dt", [D.F16, D.BF16])
def test_matmul_u16_output_rounding(dev, stream, out_dt):
    rng = np.random.default_rng(5)
    m, k, n = 320, 512, 264
    a = rand16(rng, m * k, D.F16)
    b = rand16(rng, k * n, D.F16, 0.02)
    ab, bb = upload(dev, stream, a, D.F16), upload(dev, stream, b, D.F16)
    cb = dev.alloc(m * n, out_dt)
    th.matmul(ab, bb, cb, m, k, n, D.F16, out_dt, False, stream=stream)
    got = orc.widen(cb.copy_to_host(stream), ORC[out_dt]).reshape(m, n)
    ref = orc.matmul(a, b, m, k, n, orc.F16, orc.F32)
    assert_gemm_close(got, orc.widen(orc.narrow(ref, ORC[out_dt]), ORC[out_dt]), "u16 out",
                      u16_dtype=ORC[out_dt])


@pytest.mark.parametrize("m,k,n,in_dt,out_dt,trans", [
    (1, 4096, 14336, D.F16, D.F16, False),     # decode-time projection, split K
    (8, 14336, 4096, D.BF16, D.BF16, True),    # B stored N x K, 14 slices
    (16, 4096, 4096, D.BF16, D.F32, False),
    (3, 1024, 520, D.F16, D.F32, True),        # ragged N
    (48, 2048, 1024, D.BF16, D.F32, False),    # two live 32-row blocks per wave
    (100, 1024, 768, D.F16, D.F16, True),      # whole 128-row halves
])
def test_matmul_small_m_split_k(dev, stream, m, k, n, in_dt, out_dt, trans):
    """Few 256 x 256 tiles: K is split over workgroups and the f32 partials merged."""
    rng = np.random.default_rng(m + k + n)
    a = rand16(rng, m * k, in_dt)
    b = rand16(rng, k * n, in_dt, 0.05)
    ab, bb = upload(dev, stream, a, in_dt), upload(dev, stream, b, in_dt)
    cb = dev.alloc(m * n, out_dt)
    th.matmul(ab, bb, cb, m, k, n, in_dt, out_dt, trans, stream=stream)
    raw = cb.copy_to_host(stream)
    got = raw if out_dt == D.F32 else orc.widen(raw, ORC[out_dt])
    ref = orc.matmul(a, b, m, k, n, ORC[in_dt], ORC[out_dt], b_trans=trans)
    ref32 = ref if out_dt == D.F32 else orc.widen(ref, ORC[out_dt])
    assert_gemm_close(got.reshape(m, n), ref32.reshape(m, n), f"split-K {m}x{k}x{n}",
                      u16_dtype=None if out_dt == D.F32 else ORC[out_dt])


def test_matmul_silu_mul_small_m_split_k(dev, stream):
    _swiglu_case(dev, stream, np.random.default_rng(77), 4, 4096, 2048, D.BF16, D.BF16, False)


def test_matmul_batched(dev, stream):
    rng = np.random.default_rng(6)
    bsz, m, k, n = 3, 128, 64, 96
    a = rand16(rng, bsz * m * k, D.BF16)
    b = rand16(rng, bsz * k * n, D.BF16)
    ab, bb = upload(dev, stream, a, D.BF16), upload(dev, stream, b, D.BF16)
    cb = dev.alloc(bsz * m * n, D.F32)
    th.matmul(ab, bb, cb, m, k, n, D.BF16, D.F32, False, batch=bsz, stream=stream)
    got = cb.copy_to_host(stream).reshape(bsz, m, n)
    for i in range(bsz):
        ref = orc.matmul(a[i * m * k:(i + 1) * m * k], b[i * k * n:(i + 1) * k * n], m, k, n,
                         orc.BF16)
        assert_gemm_close(got[i], ref, f"batch {i}")


def test_matmul_config2_full(dev, stream):
    """4096^3, A,B bf16 U[-1,1], C f32, rel 1e-2, every element of C."""
    M = N = K = 4096
    a = device_random(dev, stream, M * K, D.BF16, "uniform", -1.0, 1.0, 0x71130000 + 2)
    b = device_random(dev, stream, K * N, D.BF16, "uniform", -1.0, 1.0, 0x71130000 + 102)
    c = dev.alloc(M * N, D.F32)
    th.matmul(a, b, c, M, K, N, D.BF16, D.F32, False, stream=stream)
    ah, bh = a.copy_to_host(stream), b.copy_to_host(stream)
    got = c.copy_to_host(stream).reshape(M, N)
    ref = orc.matmul(ah, bh, M, K, N, orc.BF16).reshape(M, N)
    assert_gemm_close(got, ref, "config2")


def test_matmul_config3_full(dev, stream):
    """M=8192 K=4096 N=14336, f16, f32 acc, C f16, every element of C."""
    M, K, N = 8192, 4096, 14336
    a = device_random(dev, stream, M * K, D.F16, "normal", 0.0, 1.0, 0x71130000 + 3)
    b = device_random(dev, stream, K * N, D.F16, "normal", 0.0, 0.02, 0x71130000 + 103)
    c = dev.alloc(M * N, D.F16)
    th.matmul(a, b, c, M, K, N, D.F16, D.F16, False, stream=stream)
    ah, bh = a.copy_to_host(stream), b.copy_to_host(stream)
    got = orc.widen(c.copy_to_host(stream), orc.F16).reshape(M, N)
    ref = orc.matmul(ah, bh, M, K, N, orc.F16, orc.F32).reshape(M, N)
    ref16 = orc.widen(orc.narrow(ref, orc.F16), orc.F16)
    assert_gemm_close(got, ref16, "config3", u16_dtype=orc.F16)


# ---- causal mask / single-head attention ----------------------------------------------

def test_causal_mask_bit_exact(dev, stream):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((3, 70, 70)).astype(np.float32)
    xb = upload(dev, stream, x, D.F32)
    yb = dev.alloc(x.size, D.F32)
    th.causal_mask_f32(xb, yb, 70, 70, 3, stream)
    got = yb.copy_to_host(stream).reshape(3, 70, 70)
    for t in range(3):
        assert np.array_equal(got[t].view(np.uint32), orc.causal_mask_f32(x[t], 70, 70).view(np.uint32))


def test_attention_f32_golden(dev, stream, golden):
    g = golden("attention_f32.npz")
    s, d = (int(t) for t in g["sd"])
    bufs = [upload(dev, stream, g[n], D.F32) for n in "qkv"]
    ob = dev.alloc(s * d, D.F32)
    th.attention(*bufs, ob, s, d, 1, D.F32, stream)
    got = ob.copy_to_host(stream).reshape(s, d)
    assert np.abs(got - g["o"]).max() < 1e-4
    assert np.abs(got - orc.attention_f32(g["q"], g["k"], g["v"], s, d)).max() < 1e-5


@pytest.mark.parametrize("s,d,tiles,offset", [
    (200, 128, 3, 0),     # ragged last query and position blocks, three problems
    (1000, 64, 1, 0),     # many position blocks
    (1, 64, 2, 0),        # one position
    (33, 128, 2, 0),      # one full and one single-position block
    (130, 96, 2, 0),      # head_dim 96: the one-workgroup-per-query kernel
    (70, 64, 1, 1),       # views 4 bytes off 16-byte alignment: the same
])
def test_attention_f32_shapes(dev, stream, s, d, tiles, offset):
    """f32 single-head attention against the oracle on every element: the fp32 MFMA
    flash kernel (head_dim 64/128, 16-byte aligned views) sums in another order than
    the oracle's sequential loops and uses exp2, so the bound is 1e-5 absolute on
    outputs of size ~1 (the values are weighted means of V ~ N(0, 1))."""
    rng = np.random.default_rng(s * 7 + d + tiles + offset)
    q, k, v = (rng.standard_normal(tiles * s * d).astype(np.float32) for _ in range(3))
    bufs = []
    for x in (q, k, v):
        b = dev.alloc(x.size + offset, D.F32)
        b.copy_from_host(np.concatenate([np.zeros(offset, np.float32), x]), stream)
        bufs.append(b)
    ob = dev.alloc(tiles * s * d + offset, D.F32)
    ptrs = [b.as_raw_ptr() + 4 * offset for b in bufs + [ob]]
    th.attention(*ptrs, s, d, tiles, D.F32, stream)
    got = ob.copy_to_host(stream)[offset:].reshape(tiles, s, d)
    for t in range(tiles):
        sl = slice(t * s * d, (t + 1) * s * d)
        ref = orc.attention_f32(q[sl], k[sl], v[sl], s, d).reshape(s, d)
        err = np.abs(got[t] - ref).max()
        assert err < 1e-5, f"tile {t}: max err {err:.3e}"


# ---- prefill ------------------------------------------------------------------------------

def run_prefill(dev, stream, q, k, v, dtype, B, S, start, max_seq, Dh, NH, NKV):
    qb, kb, vb = (upload(dev, stream, t, dtype) for t in (q, k, v))
    ob = dev.alloc(B * S * NH * Dh, dtype)
    th.attention_prefill(qb, kb, vb, ob, B, S, start, max_seq, Dh, NH, NKV, dtype, stream)
    return orc.widen(ob.copy_to_host(stream), ORC[dtype])


def test_prefill_golden_vectors(dev, stream, golden):
    g = golden("prefill_bf16.npz")
    B, S, start, max_seq, Dh, NH, NKV = (int(t) for t in g["shape"])
    got = run_prefill(dev, stream, g["q"], g["k"], g["v"], D.BF16, B, S, start, max_seq, Dh, NH,
                      NKV)
    assert_attn_close(got, g["o"].reshape(-1), "prefill golden")


@pytest.mark.parametrize("dtype", [D.BF16, D.F16])
@pytest.mark.parametrize("B,S,start,extra,NH,NKV,Dh", [
    (1, 256, 0, 0, 2, 2, 128),     # one full query block
    (2, 300, 0, 4, 4, 1, 128),     # ragged, GQA 4:1
    (1, 100, 37, 0, 8, 2, 128),    # chunked prefill, start_pos > 0
    (1, 600, 0, 0, 2, 2, 64),      # head_dim 64 (native kernel)
    (2, 1000, 0, 0, 8, 2, 64),     # head_dim 64, GQA 4:1, grouped work order
    (1, 1500, 100, 7, 4, 4, 64),   # head_dim 64, long loop, start_pos not a multiple of 64
    (2, 300, 40, 3, 8, 2, 96),     # head_dim 96, GQA 4:1, start_pos > 0, padded
    (1, 257, 0, 0, 4, 4, 80),      # head_dim 80, padded
    (1, 70, 3, 0, 2, 1, 60),       # head_dim 60 (not a multiple of 8) -> general kernel
    (3, 1, 5, 2, 4, 4, 128),       # single query
    (1, 64, 0, 0, 2, 2, 128),      # exactly one KV block
    (1, 130, 0, 0, 2, 1, 128),     # three KV blocks, ragged query block
    (1, 1500, 100, 7, 4, 4, 128),  # long loop, start_pos not a multiple of 64
    (1, 100, 37, 3000, 8, 2, 128), # chunk of a long cache (max_seq >> start_pos + S)
    (1, 200, 300, 4000, 4, 2, 64), # head_dim 64, chunk of a long cache
    (1, 200, 300, 4000, 4, 2, 96), # padded head_dim: only live cache rows are copied
    (2, 600, 0, 0, 32, 8, 128),    # 16 (batch, kv head) units on 8 XCDs: grouped work order
    (1, 520, 64, 0, 16, 8, 128),   # 8 units, GQA 2:1, start_pos > 0
    (4, 300, 0, 0, 16, 4, 128),    # 16 units, GQA 4:1, ragged query block
    # split-KV (fewer work items than CUs, >= 16 cached blocks): parts + merge
    (1, 200, 1024, 0, 4, 2, 128),  # 4 items, 2 parts
    (2, 300, 2048, 5, 8, 2, 128),  # 32 items, 4 parts, GQA 4:1, ragged query block
    (1, 200, 1100, 0, 4, 4, 128),  # start_pos not a multiple of 64
    (1, 256, 2048, 0, 8, 2, 64),   # head_dim 64 (native parts and merge)
    (1, 256, 2048, 0, 8, 2, 80),   # on the zero-padded head_dim-80 route
    (1, 512, 7680, 0, 8, 2, 128),  # chunk after 7680 cached positions: 15 parts
])
def test_prefill_shapes(dev, stream, dtype, B, S, start, extra, NH, NKV, Dh):
    rng = np.random.default_rng(S * 7 + start)
    max_seq = start + S + extra
    q = rand16(rng, B * S * NH * Dh, dtype)
    k = rand16(rng, B * NKV * max_seq * Dh, dtype)
    v = rand16(rng, B * NKV * max_seq * Dh, dtype)
    got = run_prefill(dev, stream, q, k, v, dtype, B, S, start, max_seq, Dh, NH, NKV)
    ref = orc.attention_prefill(q, k, v, ORC[dtype], B, S, start, max_seq, Dh, NH, NKV)
    assert_attn_close(got, ref, f"prefill {dtype.name} B{B} S{S} start{start} G{NH // NKV} D{Dh}")


def test_prefill_config4_full(dev, stream, config4):
    """B=4 H=32 S=4096 D=128 bf16 causal, every output element
    against the oracle."""
    c = config4
    ob = dev.alloc(c.n, D.BF16)
    th.attention_prefill(c.q, c.k, c.v, ob, c.B, c.S, 0, c.S, c.Dh, c.H, c.H, D.BF16, stream)
    got = orc.widen(ob.copy_to_host(stream), orc.BF16).reshape(c.B, c.S, c.H, c.Dh)
    assert np.isfinite(got).all()
    for b in range(c.B):
        assert_attn_close(got[b], c.ref[b], f"config4 batch {b}")


def peaked_inputs(rng, dtype, B, S, max_seq, NH, NKV, Dh, qscale, sink):
    """Q ~ N(0, qscale^2); with `sink`, every query leans on one direction u and key 0
    of every kv head is 3u*sqrt(D), so that key's score sits ~9 above a typical score
    and it carries a large share of every row's probability mass (an attention sink)."""
    q = rng.standard_normal((B, S, NH, Dh)) * qscale
    k = rng.standard_normal((B, NKV, max_seq, Dh))
    v = rng.standard_normal((B, NKV, max_seq, Dh))
    if sink:
        u = rng.standard_normal(Dh)
        u /= np.linalg.norm(u)
        q += 3.0 * u
        k[:, :, 0, :] = 3.0 * np.sqrt(Dh) * u
    return tuple(orc.narrow(t.astype(np.float32).reshape(-1), ORC[dtype]) for t in (q, k, v))


PEAKED = {"q2.5": (2.5, False), "q4": (4.0, False), "sink": (1.0, True), "sink_q2.5": (2.5, True)}


@pytest.mark.parametrize("dtype", [D.BF16, D.F16])
@pytest.mark.parametrize("kind", list(PEAKED))
@pytest.mark.parametrize("B,S,start,NH,NKV,Dh", [
    (1, 1024, 0, 4, 2, 128),     # 4 query blocks, GQA 2:1
    (1, 600, 0, 4, 4, 64),       # native head_dim 64
    (1, 300, 1500, 8, 2, 128),   # a chunk after 1500 cached positions: split-KV parts + merge
])
def test_prefill_peaked(dev, stream, dtype, kind, B, S, start, NH, NKV, Dh):
    """Peaked scores (Q scaled x2.5, x4) and a dominant early key: the inputs for which
    the kernel applies the rounding residual of its 16-bit P (one key holding a large
    share of a row's mass so far), checked on the kernel itself."""
    qscale, sink = PEAKED[kind]
    rng = np.random.default_rng(S + start + int(qscale * 10) + sink)
    max_seq = start + S
    q, k, v = peaked_inputs(rng, dtype, B, S, max_seq, NH, NKV, Dh, qscale, sink)
    got = run_prefill(dev, stream, q, k, v, dtype, B, S, start, max_seq, Dh, NH, NKV)
    ref = orc.attention_prefill(q, k, v, ORC[dtype], B, S, start, max_seq, Dh, NH, NKV)
    assert_attn_close(got, ref, f"prefill {kind} {dtype.name} S{S} start{start} D{Dh}")


@pytest.mark.parametrize("kind", ["q4", "sink_q2.5"])
def test_prefill_config4_peaked(dev, stream, kind):
    """Config-4 shape (B=4 H=32 S=4096 D=128 bf16) with peaked queries or an attention
    sink; eight (batch, head) pairs checked in full."""
    B, H, S, Dh = 4, 32, 4096, 128
    qscale, sink = PEAKED[kind]
    rng = np.random.default_rng(0x4444 + int(qscale * 10))
    q, k, v = peaked_inputs(rng, D.BF16, B, S, S, H, H, Dh, qscale, sink)
    got = run_prefill(dev, stream, q, k, v, D.BF16, B, S, 0, S, Dh, H, H).reshape(B, S, H, Dh)
    for bh in (0, 17, 38, 63, 64, 95, 110, 127):
        b, h = divmod(bh, H)
        ref = orc.attention_prefill(q, k, v, orc.BF16, B, S, 0, S, Dh, H, H, bh0=bh, nbh=1)
        assert_attn_close(got[b, :, h], ref.reshape(B, S, H, Dh)[b, :, h],
                          f"config4 {kind} bh={bh}")


@pytest.mark.parametrize("dtype", [D.BF16, D.F16])
def test_prefill_repeat_bit_identical(dev, stream, dtype):
    """Repeated launches on the same inputs give the same bits.  The loop is hand-written
    assembly, so a missing wait state shows up as run-to-run drift: before the
    transcendental-forwarding fix, 1.6% of config-4 outputs moved by 1-2 ulp between
    launches (all in query blocks that stream K/V inside the loop)."""
    B, H, S, Dh = 1, 32, 2048, 128
    n = B * S * H * Dh
    qb = device_random(dev, stream, n, dtype, "normal", 0.0, 1.0, 0x5151)
    kb = device_random(dev, stream, n, dtype, "normal", 0.0, 1.0, 0x5152)
    vb = device_random(dev, stream, n, dtype, "normal", 0.0, 1.0, 0x5153)
    ob = dev.alloc(n, dtype)
    outs = []
    for _ in range(4):
        th.attention_prefill(qb, kb, vb, ob, B, S, 0, S, Dh, H, H, dtype, stream)
        outs.append(ob.copy_to_host(stream).copy())
    for i, o in enumerate(outs[1:], 1):
        nd = int(np.count_nonzero(o != outs[0]))
        assert nd == 0, f"launch {i}: {nd} of {n} outputs differ from launch 0"


# ---- decode --------------------------------------------------------------------------------

def run_decode(dev, stream, q, k, v, dtype, B, L, max_seq, Dh, NH, NKV, workspace=False):
    qb, kb, vb = (upload(dev, stream, t, dtype) for t in (q, k, v))
    ob = dev.alloc(B * NH * Dh, dtype)
    ws, wsz = None, 0
    if workspace:
        wsz = th.attention_decode_workspace_size(B, L, Dh, NH, NKV)
        ws = dev.alloc(max(1, wsz // 4), D.F32)
    th.attention_decode(qb, kb, vb, ob, B, L, max_seq, Dh, NH, NKV, dtype, ws, wsz, stream)
    return orc.widen(ob.copy_to_host(stream), ORC[dtype])


def test_decode_golden_vectors(dev, stream, golden):
    g = golden("decode_bf16.npz")
    B, L, max_seq, Dh, NH, NKV = (int(t) for t in g["shape"])
    got = run_decode(dev, stream, g["q"], g["k"], g["v"], D.BF16, B, L, max_seq, Dh, NH, NKV)
    assert_attn_close(got, g["o"].reshape(-1), "decode golden")


@pytest.mark.parametrize("dtype", [D.BF16, D.F16])
@pytest.mark.parametrize("B,L,extra,NH,NKV,Dh,ws", [
    (2, 300, 20, 8, 2, 128, False),
    (1, 1, 0, 4, 4, 128, True),       # one position
    (3, 513, 7, 16, 1, 128, True),    # G=16, chunk boundary + 1
    (2, 1024, 0, 8, 8, 128, False),   # MHA
    (2, 777, 0, 4, 2, 64, False),     # head_dim 64 (native kernel), split
    (1, 9000, 40, 8, 1, 64, True),    # head_dim 64, G=8, rows past seq_len not read
    (64, 600, 0, 8, 8, 96, False),    # head_dim 96, unsplit
    (1, 300, 0, 4, 2, 60, False),     # head_dim 60 (not a multiple of 8) -> general kernel
    (1, 200, 0, 6, 2, 128, False),   # G=3 -> general kernel
    (1, 4500, 3, 4, 2, 128, False),   # 9 chunks: one batch of 8 partials + 1 in the merge
    (1, 66000, 0, 2, 1, 128, True),   # 129 chunks: the merge stages partials in two passes
    (16, 4196, 0, 16, 8, 128, False),  # 128 items x 9 chunks: splits of several chunks each
    (64, 1500, 0, 8, 8, 128, True),   # 512 items: one workgroup per item walks all chunks
    (1, 5000, 9, 8, 2, 64, True),     # head_dim 64, split, caller's workspace (128-wide records)
    (64, 1100, 0, 32, 8, 64, False),  # head_dim 64, 512 items, unsplit
    (3, 2100, 5, 16, 1, 64, True),    # head_dim 64, G=16
    (2, 700, 0, 8, 4, 80, False),     # head_dim 80: zero-padded to 128
])
def test_decode_shapes(dev, stream, dtype, B, L, extra, NH, NKV, Dh, ws):
    rng = np.random.default_rng(L * 3 + NH)
    max_seq = L + extra
    q = rand16(rng, B * NH * Dh, dtype)
    k = rand16(rng, B * NKV * max_seq * Dh, dtype)
    v = rand16(rng, B * NKV * max_seq * Dh, dtype)
    got = run_decode(dev, stream, q, k, v, dtype, B, L, max_seq, Dh, NH, NKV, ws)
    ref = orc.attention_decode(q, k, v, ORC[dtype], B, L, max_seq, Dh, NH, NKV)
    assert_attn_close(got, ref, f"decode {dtype.name} B{B} L{L} G{NH // NKV} D{Dh}")


def test_decode_config5_full(dev, stream):
    """B=64, NH=32, NKV=8, L=8192, D=128 bf16, all outputs."""
    B, NH, NKV, L, Dh = 64, 32, 8, 8192, 128
    qb = device_random(dev, stream, B * NH * Dh, D.BF16, "normal", 0.0, 1.0, 0x71130000 + 5)
    kb = device_random(dev, stream, B * NKV * L * Dh, D.BF16, "normal", 0.0, 1.0, 0x71130000 + 105)
    vb = device_random(dev, stream, B * NKV * L * Dh, D.BF16, "normal", 0.0, 1.0, 0x71130000 + 205)
    ob = dev.alloc(B * NH * Dh, D.BF16)
    th.attention_decode(qb, kb, vb, ob, B, L, L, Dh, NH, NKV, D.BF16, stream=stream)
    q, k, v = (b.copy_to_host(stream) for b in (qb, kb, vb))
    got = orc.widen(ob.copy_to_host(stream), orc.BF16)
    ref = orc.attention_decode(q, k, v, orc.BF16, B, L, L, Dh, NH, NKV)
    assert_attn_close(got, ref, "config5")


def test_decode_matches_last_prefill_row(dev, stream):
    rng = np.random.default_rng(21)
    B, NH, NKV, Dh, L = 2, 8, 2, 128, 700
    q = rand16(rng, B * NH * Dh, D.BF16)
    k = rand16(rng, B * NKV * L * Dh, D.BF16)
    v = rand16(rng, B * NKV * L * Dh, D.BF16)
    od = run_decode(dev, stream, q, k, v, D.BF16, B, L, L, Dh, NH, NKV)
    op = run_prefill(dev, stream, q, k, v, D.BF16, B, 1, L - 1, L, Dh, NH, NKV)
    assert_attn_close(od, op, "decode vs prefill last row")


# ---- rms_norm (row RMSNorm, tile.rs:2063) ------------------------------------------------

def test_rms_norm_golden_vectors(dev, stream, golden):
    g = golden("rms_norm_f32.npz")
    x = g["x"]
    rows, cols = x.shape
    xb, yb = upload(dev, stream, x, D.F32), dev.alloc(x.size, D.F32)
    th.rms_norm(xb, yb, rows, cols, float(g["eps"][0]), D.F32, stream)
    assert_softmax_close(yb.copy_to_host(stream).reshape(rows, cols), g["y"], "rms_norm golden")


@pytest.mark.parametrize("rows,cols,eps", [(8192, 1024, 1e-6), (3, 1000, 1e-5), (7, 1, 1e-5),
                                           (12345, 256, 1e-6), (5, 5003, 0.0), (20001, 128, 1e-5),
                                           (33, 4096, 1e-6), (2, 77, 0.5)])
def test_rms_norm_f32_shapes(dev, stream, rows, cols, eps):
    rng = np.random.default_rng(rows * 17 + cols)
    x = (rng.standard_normal((rows, cols)) * 1.5).astype(np.float32)
    xb, yb = upload(dev, stream, x, D.F32), dev.alloc(x.size, D.F32)
    th.rms_norm(xb, yb, rows, cols, eps, D.F32, stream)
    assert_softmax_close(yb.copy_to_host(stream).reshape(rows, cols),
                         orc.rms_norm(x, rows, cols, eps), f"rms_norm {rows}x{cols}")


@pytest.mark.parametrize("dtype", [D.F16, D.BF16])
@pytest.mark.parametrize("rows,cols", [(64, 2048), (3, 100), (4, 8192), (17003, 512)])
def test_rms_norm_u16(dev, stream, dtype, rows, cols):
    rng = np.random.default_rng(cols + 5)
    x = rand16(rng, rows * cols, dtype, 2.0)
    xb, yb = upload(dev, stream, x, dtype), dev.alloc(x.size, dtype)
    th.rms_norm(xb, yb, rows, cols, 1e-6, dtype, stream)
    y = orc.widen(yb.copy_to_host(stream), ORC[dtype])
    ref = orc.widen(orc.rms_norm(x, rows, cols, 1e-6, ORC[dtype]), ORC[dtype])
    assert_within_ulp16(y, ref, ORC[dtype], 1.0, f"rms_norm {dtype.name} {rows}x{cols}")


@pytest.mark.parametrize("dtype,rows,cols", [(D.F32, 64, 131072), (D.F32, 2, 70000),
                                             (D.BF16, 300, 16384), (D.BF16, 260, 32768),
                                             (D.F16, 5, 100003), (D.BF16, 3, 12289)])
def test_rms_norm_long_rows(dev, stream, dtype, rows, cols):
    """Rows beyond one wave's registers: one workgroup per row (enough rows), else chunk
    sums of squares merged per row; ragged rows take the scalar form."""
    rng = np.random.default_rng(rows + cols)
    eps = 1e-6
    if dtype == D.F32:
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        xb = upload(dev, stream, x, D.F32)
        yb = dev.alloc(x.size, D.F32)
        th.rms_norm(xb, yb, rows, cols, eps, D.F32, stream)
        assert_softmax_close(yb.copy_to_host(stream).reshape(rows, cols),
                             orc.rms_norm(x, rows, cols, eps), f"rms_norm {rows}x{cols}")
    else:
        x = rand16(rng, rows * cols, dtype, 1.0)
        xb = upload(dev, stream, x, dtype)
        yb = dev.alloc(x.size, dtype)
        th.rms_norm(xb, yb, rows, cols, eps, dtype, stream)
        y = orc.widen(yb.copy_to_host(stream), ORC[dtype])
        ref = orc.rms_norm(orc.widen(x, ORC[dtype]), rows, cols, eps)
        assert_within_ulp16(y, ref, ORC[dtype], 1.0, f"rms_norm {dtype.name} {rows}x{cols}")


def test_rms_norm_in_place_and_errors(dev, stream):
    rng = np.random.default_rng(8)
    x = rng.standard_normal((16, 1024)).astype(np.float32)
    b = upload(dev, stream, x, D.F32)
    th.rms_norm(b, b, 16, 1024, 1e-6, D.F32, stream)
    assert_softmax_close(b.copy_to_host(stream).reshape(16, 1024), orc.rms_norm(x, 16, 1024, 1e-6))
    with pytest.raises(th.HalError):
        th.rms_norm(b, b, 16, 1024, -1.0, D.F32, stream)


# ---- matmul with the SiLU*Mul epilogue (matmul -> silu -> mul chain) ---------------------

def _swiglu_case(dev, stream, rng, m, k, n, in_dt, out_dt, trans, batch=1):
    a = rand16(rng, batch * m * k, in_dt) if in_dt != D.F32 else \
        rng.standard_normal(batch * m * k).astype(np.float32)
    b = (rand16(rng, batch * k * n, in_dt, 0.1) if in_dt != D.F32 else
         (rng.standard_normal(batch * k * n) * 0.1).astype(np.float32))
    u32 = rng.standard_normal(batch * m * n).astype(np.float32)
    u = u32 if out_dt == D.F32 else orc.narrow(u32, ORC[out_dt])
    ab, bb, ub = (upload(dev, stream, a, in_dt), upload(dev, stream, b, in_dt),
                  upload(dev, stream, u, out_dt))
    cb = dev.alloc(batch * m * n, out_dt)
    th.matmul_silu_mul(ab, bb, ub, cb, m, k, n, in_dt, out_dt, trans, batch, stream=stream)
    raw = cb.copy_to_host(stream)
    got = (raw if out_dt == D.F32 else orc.widen(raw, ORC[out_dt])).reshape(batch, m, n)
    for i in range(batch):
        ref = orc.matmul_silu_mul(a[i * m * k:(i + 1) * m * k], b[i * k * n:(i + 1) * k * n],
                                  u[i * m * n:(i + 1) * m * n], m, k, n, ORC[in_dt], ORC[out_dt],
                                  b_trans=trans)
        ref32 = ref if out_dt == D.F32 else orc.widen(ref, ORC[out_dt])
        assert_gemm_close(got[i], ref32.reshape(m, n), f"swiglu {m}x{k}x{n} batch {i}",
                          u16_dtype=None if out_dt == D.F32 else ORC[out_dt])


def test_matmul_silu_mul_golden_vectors(dev, stream, golden):
    g = golden("swiglu_bf16.npz")
    m, k, n = (int(v) for v in g["mkn"])
    ab, bb = upload(dev, stream, g["a"], D.BF16), upload(dev, stream, g["b"], D.BF16)
    ub, cb = upload(dev, stream, g["up"], D.F32), dev.alloc(m * n, D.F32)
    th.matmul_silu_mul(ab, bb, ub, cb, m, k, n, D.BF16, D.F32, False, stream=stream)
    assert_gemm_close(cb.copy_to_host(stream).reshape(m, n), g["c"], "swiglu golden")


@pytest.mark.parametrize("m,k,n,in_dt,out_dt,trans", [
    (512, 512, 768, D.BF16, D.F32, False),    # LDS-DMA pipeline
    (256, 1024, 512, D.F16, D.F16, True),     # generated-assembly program, B stored N x K
    (512, 384, 768, D.BF16, D.BF16, False),   # generated-assembly program (whole tiles)
    (256, 512, 256, D.F16, D.BF16, False),    # same, f16 operands, bf16 C and UP
    (512, 256, 256, D.BF16, D.F16, True),     # same, B stored N x K
    (512, 96, 256, D.BF16, D.BF16, False),    # LDS-DMA pipeline, 3 stages of K
    (512, 80, 256, D.BF16, D.BF16, False),    # register-staged MFMA (K % 32 != 0)
    (300, 72, 136, D.F16, D.F32, False),      # ragged MFMA tiles
    (300, 128, 136, D.F16, D.F16, False),     # LDS-DMA pipeline, tiles cut by M and N
    (200, 256, 328, D.BF16, D.F32, True),     # same, B stored N x K
    (64, 33, 40, D.BF16, D.F32, True),        # FMA fallback (K % 8 != 0)
    (96, 64, 80, D.F32, D.F32, False),        # f32 operands
])
def test_matmul_silu_mul_shapes(dev, stream, m, k, n, in_dt, out_dt, trans):
    _swiglu_case(dev, stream, np.random.default_rng(m + 3 * k + 5 * n), m, k, n, in_dt, out_dt,
                 trans)


def test_matmul_silu_mul_unaligned_output(dev, stream):
    """UP and C one element past a 16-byte boundary: the 16-byte epilogue of the DMA
    pipeline does not apply and the register-staged kernel handles the shape."""
    rng = np.random.default_rng(91)
    m = k = n = 256
    a, b = rand16(rng, m * k, D.BF16), rand16(rng, k * n, D.BF16, 0.1)
    u = orc.narrow(rng.standard_normal(m * n).astype(np.float32), orc.BF16)
    ab, bb = upload(dev, stream, a, D.BF16), upload(dev, stream, b, D.BF16)
    ub = upload(dev, stream, np.concatenate([np.zeros(1, u.dtype), u]), D.BF16)
    cb = dev.alloc(m * n + 1, D.BF16)
    th.matmul_silu_mul(ab, bb, ub.as_raw_ptr() + 2, cb.as_raw_ptr() + 2, m, k, n, D.BF16,
                       D.BF16, False, stream=stream)
    got = orc.widen(cb.copy_to_host(stream)[1:], orc.BF16).reshape(m, n)
    ref = orc.matmul_silu_mul(a, b, u, m, k, n, orc.BF16, orc.BF16)
    assert_gemm_close(got, orc.widen(ref, orc.BF16).reshape(m, n), "swiglu unaligned",
                      u16_dtype=orc.BF16)


def test_matmul_silu_mul_batched(dev, stream):
    _swiglu_case(dev, stream, np.random.default_rng(77), 256, 128, 256, D.F16, D.F16, False,
                 batch=3)


def test_matmul_silu_mul_whole_tiles_batched(dev, stream):
    """Whole tiles over a batch of two (the assembly program; UP and C step by the
    batch stride together)."""
    _swiglu_case(dev, stream, np.random.default_rng(78), 256, 256, 512, D.BF16, D.BF16, False,
                 batch=2)


@pytest.mark.parametrize("trans", [False, True])
@pytest.mark.parametrize("in_dt", [D.BF16, D.F16])
@pytest.mark.parametrize("out_dt", [D.BF16, D.F16])
def test_matmul_silu_mul_whole_tiles_every_variant(dev, stream, trans, in_dt, out_dt):
    """Each of the assembly program's eight SiLU*Mul variants (operand dtype x C/UP dtype
    x B layout) on two 256 x 256 tiles with K = 384 (12 steps of 32)."""
    _swiglu_case(dev, stream, np.random.default_rng(90 + 4 * trans + 2 * (in_dt == D.F16) +
                                                    (out_dt == D.F16)),
                 256, 384, 512, in_dt, out_dt, trans)


def test_matmul_silu_mul_saturated_gate(dev, stream):
    """Gate values far past the exponential's range (|A.B| up to ~200): silu(x) -> x for
    large x and -> -0 for large negative x, with no NaN from inf / inf."""
    rng = np.random.default_rng(79)
    m, k, n = 256, 256, 256
    a = rand16(rng, m * k, D.F16, 4.0)
    b = rand16(rng, k * n, D.F16, 4.0)
    u = orc.narrow(rng.standard_normal(m * n).astype(np.float32), orc.F16)
    ab, bb, ub = upload(dev, stream, a, D.F16), upload(dev, stream, b, D.F16), upload(dev, stream, u, D.F16)
    cb = dev.alloc(m * n, D.F16)
    th.matmul_silu_mul(ab, bb, ub, cb, m, k, n, D.F16, D.F16, False, stream=stream)
    got = orc.widen(cb.copy_to_host(stream), orc.F16).reshape(m, n)
    ref = orc.widen(orc.matmul_silu_mul(a, b, u, m, k, n, orc.F16, orc.F16), orc.F16).reshape(m, n)
    assert np.isfinite(got).all()
    g = orc.matmul(a, b, m, k, n, orc.F16, orc.F32).reshape(m, n)
    assert np.abs(g).max() > 60
    assert_gemm_close(got, ref, "swiglu saturated", u16_dtype=orc.F16)


def test_matmul_silu_mul_config3_subset(dev, stream):
    """The MLP shape of BASELINE config 3 with the gate epilogue: 96 rows checked."""
    m, k, n = 8192, 4096, 14336
    a = device_random(dev, stream, m * k, D.F16, "normal", 0.0, 1.0, 0x71130000 + 3)
    b = device_random(dev, stream, k * n, D.F16, "normal", 0.0, 0.02, 0x71130000 + 103)
    u = device_random(dev, stream, m * n, D.F16, "normal", 0.0, 1.0, 0x71130000 + 203)
    c = dev.alloc(m * n, D.F16)
    th.matmul_silu_mul(a, b, u, c, m, k, n, D.F16, D.F16, False, stream=stream)
    ah = a.copy_to_host(stream).reshape(m, k)
    bh, uh = b.copy_to_host(stream), u.copy_to_host(stream)
    got = orc.widen(c.copy_to_host(stream), orc.F16).reshape(m, n)
    for r0 in (0, 4064, 8160):
        ref = orc.matmul_silu_mul(np.ascontiguousarray(ah[r0:r0 + 32]), bh,
                                  uh.reshape(m, n)[r0:r0 + 32], 32, k, n, orc.F16, orc.F16)
        assert_gemm_close(got[r0:r0 + 32], orc.widen(ref, orc.F16).reshape(32, n),
                          f"config3 swiglu rows {r0}", u16_dtype=orc.F16)

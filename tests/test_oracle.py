"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the parity checker.

Each check is independent of the oracle's own formulas: golden vectors from an
independent float64 implementation (tests/golden), exhaustive conversion
sweeps, closed forms and invariants, and bit-exact brute force on
integer-valued inputs.  CPU only.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc

F32, F16, BF16 = orc.F32, orc.F16, orc.BF16


def bits_to_f32(u16: np.ndarray) -> np.ndarray:
    return (u16.astype(np.uint32) << 16).view(np.float32)


# ---- 16-bit conversions ---------------------------------------------------------------

def test_bf16_widen_is_exact_shift():
    allp = np.arange(65536, dtype=np.uint16)
    w = orc.widen(allp, BF16)
    assert np.array_equal(w.view(np.uint32), allp.astype(np.uint32) << 16)


def test_bf16_round_trip_all_patterns():
    allp = np.arange(65536, dtype=np.uint16)
    back = orc.narrow(orc.widen(allp, BF16), BF16)
    nan = np.isnan(bits_to_f32(allp))
    assert np.array_equal(back[~nan], allp[~nan])
    assert np.isnan(bits_to_f32(back[nan])).all()


def test_f16_matches_numpy_float16_all_patterns():
    allp = np.arange(65536, dtype=np.uint16)
    w = orc.widen(allp, F16)
    ref = allp.view(np.float16).astype(np.float32)
    same = (w.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(w) & np.isnan(ref))
    assert same.all()


def test_f32_to_f16_matches_numpy_rounding():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 10,
        rng.standard_normal(50000).astype(np.float32) * 1e-6,   # subnormal range of f16
        rng.standard_normal(50000).astype(np.float32) * 7e4,    # overflow range
        np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65520, 65519.99, 2 ** -25, 2 ** -24,
                  3 * 2 ** -26], np.float32),
    ])
    got = orc.narrow(x, F16)
    with np.errstate(over="ignore"):     # the overflow range rounds to inf on purpose
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_bf16_is_nearest_even():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(300000) * np.exp(rng.uniform(-30, 30, 300000))).astype(np.float32)
    x = np.concatenate([x, np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8)],
                                    np.float32)])
    r = orc.narrow(x, BF16)
    rv = bits_to_f32(r).astype(np.float64)
    xv = x.astype(np.float64)
    up = bits_to_f32((r.astype(np.int32) + 1).astype(np.uint16)).astype(np.float64)
    dn = bits_to_f32((r.astype(np.int32) - 1).astype(np.uint16)).astype(np.float64)
    d0 = np.abs(xv - rv)
    ok = np.isfinite(up) & np.isfinite(dn) & (np.abs(r.astype(np.int32) & 0x7fff) > 1)
    assert (d0[ok] <= np.abs(xv - up)[ok]).all() and (d0[ok] <= np.abs(xv - dn)[ok]).all()
    tie = ok & ((d0 == np.abs(xv - up)) | (d0 == np.abs(xv - dn)))
    assert ((r[tie] & 1) == 0).all()
    # the explicit ties: 1 + 2^-8 -> 1.0 (even), 1 + 3*2^-8 -> 1 + 2^-6... rounds to even
    assert bits_to_f32(r[-3:-2])[0] == 1.0
    assert bits_to_f32(r[-1:])[0] == -1.0


# ---- softmax -------------------------------------------------------------------------

def test_softmax_golden(golden):
    g = golden("softmax_f32.npz")
    y = orc.softmax(g["x"], *g["x"].shape)
    assert np.allclose(y, g["y"], rtol=2e-6, atol=0)


def test_softmax_invariants():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 1000)) * 2).astype(np.float32)
    y = orc.softmax(x, 64, 1000)
    assert np.allclose(y.sum(axis=1), 1.0, atol=2e-6)
    y2 = orc.softmax((x + 3.0).astype(np.float32), 64, 1000)
    assert np.allclose(y, y2, rtol=2e-5, atol=1e-9)
    c = np.full((2, 128), -7.25, np.float32)
    assert np.all(orc.softmax(c, 2, 128) == np.float32(1 / 128))
    one_hot = np.zeros((1, 16), np.float32)
    one_hot[0, 5] = 1000.0
    yh = orc.softmax(one_hot, 1, 16)
    assert yh[0, 5] == 1.0 and np.all(np.delete(yh[0], 5) == 0.0)


def test_softmax_u16_is_f32_softmax_rounded():
    rng = np.random.default_rng(4)
    x = orc.narrow((rng.standard_normal((8, 256)) * 2).astype(np.float32), BF16)
    y = orc.softmax(x, 8, 256, BF16)
    ref = orc.softmax(orc.widen(x, BF16), 8, 256)
    assert np.array_equal(y, orc.narrow(ref, BF16))


# ---- rms_norm ------------------------------------------------------------------------------

def test_rms_norm_golden(golden):
    g = golden("rms_norm_f32.npz")
    x = g["x"]
    y = orc.rms_norm(x, *x.shape, float(g["eps"][0]))
    assert np.allclose(y, g["y"], rtol=2e-6, atol=0)


def test_rms_norm_closed_forms():
    eps = 1e-5
    c = np.full((1, 64), -0.75, np.float32)  # constant row -> c / sqrt(c^2 + eps)
    assert np.allclose(orc.rms_norm(c, 1, 64, eps), -0.75 / np.sqrt(0.5625 + eps), rtol=1e-7)
    h = np.zeros((1, 100), np.float32)       # one-hot row: v * rsqrt(v^2/100 + eps)
    h[0, 7] = 5.0
    yh = orc.rms_norm(h, 1, 100, eps)
    assert np.isclose(yh[0, 7], 5.0 / np.sqrt(25.0 / 100 + eps), rtol=1e-7)
    assert np.all(np.delete(yh[0], 7) == 0.0)


def test_rms_norm_invariants():
    rng = np.random.default_rng(21)
    x = rng.standard_normal((32, 300)).astype(np.float32)
    # eps = 0: every row has mean(y^2) = 1, and scaling by a power of two cancels
    y0 = orc.rms_norm(x, 32, 300, 0.0)
    assert np.allclose((y0.astype(np.float64) ** 2).mean(axis=1), 1.0, rtol=1e-6)
    y4 = orc.rms_norm((x * -4.0).astype(np.float32), 32, 300, 0.0)
    assert np.array_equal(y4, -y0)
    # eps > 0: mean(y^2) = mean / (mean + eps)
    eps = 0.25
    y = orc.rms_norm(x, 32, 300, eps)
    ms = (x.astype(np.float64) ** 2).mean(axis=1)
    assert np.allclose((y.astype(np.float64) ** 2).mean(axis=1), ms / (ms + eps), rtol=1e-6)


def test_rms_norm_u16_is_f32_rms_norm_rounded():
    rng = np.random.default_rng(22)
    x = orc.narrow(rng.standard_normal((8, 192)).astype(np.float32), BF16)
    y = orc.rms_norm(x, 8, 192, 1e-6, BF16)
    ref = orc.rms_norm(orc.widen(x, BF16), 8, 192, 1e-6)
    diff = np.abs(y.astype(np.int32) - orc.narrow(ref, BF16).astype(np.int32))
    assert diff.max() <= 1  # f64 -> f32 -> bf16 vs f64 -> bf16 may differ by one ulp


# ---- silu * mul ----------------------------------------------------------------------------

def _rope_angle(pos, i, cols):
    """pos * 10000^(-2i/cols) in float64 (the rotation angle of pair i)."""
    return pos * 10000.0 ** (-2.0 * i / cols)


def test_rope_position_zero_is_identity():
    x = np.random.default_rng(31).standard_normal((5, 48)).astype(np.float32)
    assert np.array_equal(orc.rope(x, 5, 48, 0), x)


def test_rope_unit_pairs_follow_cos_sin():
    cols, pos = 32, 5
    e0 = np.zeros((1, cols), np.float32)
    e0[0, 0::2] = 1.0   # every pair (1, 0)
    e1 = np.zeros((1, cols), np.float32)
    e1[0, 1::2] = 1.0   # every pair (0, 1)
    t = _rope_angle(pos, np.arange(cols // 2), cols)
    y0, y1 = orc.rope(e0, 1, cols, pos)[0], orc.rope(e1, 1, cols, pos)[0]
    # (1, 0) -> (cos t, sin t); (0, 1) -> (-sin t, cos t).  The frequency is
    # formed in f32, so the angle carries ~1e-7 relative error.
    assert np.allclose(y0[0::2], np.cos(t), atol=4e-6) and np.allclose(y0[1::2], np.sin(t), atol=4e-6)
    assert np.allclose(y1[0::2], -np.sin(t), atol=4e-6) and np.allclose(y1[1::2], np.cos(t), atol=4e-6)


def test_rope_keeps_pair_norms_and_composes():
    rng = np.random.default_rng(32)
    x = rng.standard_normal((6, 64)).astype(np.float32)
    y = orc.rope(x, 6, 64, 37).astype(np.float64)
    xd = x.astype(np.float64)
    n_in = xd[:, 0::2] ** 2 + xd[:, 1::2] ** 2
    n_out = y[:, 0::2] ** 2 + y[:, 1::2] ** 2
    assert np.allclose(n_out, n_in, rtol=1e-6)
    # a rotation group: rope(rope(x, a), b) = rope(x, a + b)
    ab = orc.rope(orc.rope(x, 6, 64, 3), 6, 64, 4)
    assert np.allclose(ab, orc.rope(x, 6, 64, 7), atol=2e-6)


def test_rope_u16_is_f32_rope_rounded():
    rng = np.random.default_rng(33)
    for dt in (orc.BF16, orc.F16):
        x = orc.narrow(rng.standard_normal(2 * 128).astype(np.float32), dt)
        y = orc.rope(x, 2, 128, 1000, dt)
        ref = orc.narrow(orc.rope(orc.widen(x, dt), 2, 128, 1000), dt)
        assert np.array_equal(y, ref)


def test_silu_mul_closed_forms():
    x = np.array([0.0, 1.0, -1.0, 3.5, -3.5, 40.0, -40.0, 100.0], np.float32)
    ones = np.ones_like(x)
    s = orc.silu_mul(x, ones).astype(np.float64)
    assert s[0] == 0.0
    assert np.allclose(s[1] - s[2], 1.0, rtol=1e-7) and np.allclose(s[3] - s[4], 3.5, rtol=1e-7)
    assert s[5] == np.float32(40.0) and abs(s[6]) < 1e-15 and s[7] == 100.0
    assert np.isclose(s[1], 1.0 / (1.0 + np.exp(-1.0)), rtol=1e-7)
    up = np.array([2.0, -3.0, 0.5, 1.0, 1.0, 1.0, 1.0, 0.0], np.float32)
    assert np.allclose(orc.silu_mul(x, up), s * up, rtol=1e-7)


def test_matmul_silu_mul_golden(golden):
    g = golden("swiglu_bf16.npz")
    m, k, n = g["mkn"]
    c = orc.matmul_silu_mul(g["a"], g["b"], g["up"], m, k, n, BF16, F32)
    rms = np.sqrt(np.mean(g["c"].astype(np.float64) ** 2))
    assert np.abs(c - g["c"]).max() <= 1e-5 * rms


def test_matmul_silu_mul_is_silu_mul_of_matmul():
    rng = np.random.default_rng(23)
    m, k, n = 40, 24, 56
    a = orc.narrow(rng.standard_normal((m, k)).astype(np.float32), F16)
    b = orc.narrow(rng.standard_normal((n, k)).astype(np.float32) * 0.2, F16)
    up = orc.narrow(rng.standard_normal((m, n)).astype(np.float32), F16)
    c = orc.matmul_silu_mul(a, b, up, m, k, n, F16, F16, b_trans=True)
    acc = orc.matmul(a, b, m, k, n, F16, F32, b_trans=True)
    ref = orc.silu_mul(acc, orc.widen(up, F16).reshape(m, n))
    diff = np.abs(c.astype(np.int32) - orc.narrow(ref, F16).astype(np.int32))
    assert diff.max() <= 1
    rows = orc.matmul_silu_mul(a, b, up, m, k, n, F16, F16, b_trans=True, row0=13, nrows=9)
    assert np.array_equal(rows, c[13:22])


# ---- matmul --------------------------------------------------------------------------------

def test_matmul_golden_bf16(golden):
    g = golden("matmul_bf16.npz")
    m, k, n = g["mkn"]
    c = orc.matmul(g["a"], g["b"], m, k, n, BF16)
    rms = np.sqrt(np.mean(g["c"].astype(np.float64) ** 2))
    assert np.abs(c - g["c"]).max() <= 1e-5 * rms


def test_matmul_golden_f16_transposed(golden):
    g = golden("matmul_f16_t.npz")
    m, k, n = g["mkn"]
    c = orc.matmul(g["a"], g["b"], m, k, n, F16, b_trans=True)
    rms = np.sqrt(np.mean(g["c"].astype(np.float64) ** 2))
    assert np.abs(c - g["c"]).max() <= 1e-5 * rms


@pytest.mark.parametrize("trans", [False, True])
def test_matmul_integer_inputs_bit_exact(trans):
    rng = np.random.default_rng(5)
    m, k, n = 37, 200, 29
    a = rng.integers(-4, 5, (m, k)).astype(np.float32)
    b = rng.integers(-4, 5, (n, k) if trans else (k, n)).astype(np.float32)
    ref = a.astype(np.int64) @ (b.T if trans else b).astype(np.int64)
    c = orc.matmul(orc.narrow(a, BF16), orc.narrow(b, BF16), m, k, n, BF16, b_trans=trans)
    assert np.array_equal(c, ref.astype(np.float32))
    c32 = orc.matmul(a, b, m, k, n, F32, b_trans=trans)
    assert np.array_equal(c32, ref.astype(np.float32))


def test_matmul_identity_and_permutation():
    rng = np.random.default_rng(6)
    a = (rng.standard_normal((24, 24))).astype(np.float32)
    eye = np.eye(24, dtype=np.float32)
    assert np.array_equal(orc.matmul(a, eye, 24, 24, 24, F32), a)
    perm = np.eye(24, dtype=np.float32)[rng.permutation(24)]
    assert np.array_equal(orc.matmul(perm, a, 24, 24, 24, F32), perm @ a)


def test_matmul_row_subset_matches_full():
    rng = np.random.default_rng(7)
    a = orc.narrow(rng.standard_normal((50, 64)).astype(np.float32), F16)
    b = orc.narrow(rng.standard_normal((64, 40)).astype(np.float32), F16)
    full = orc.matmul(a, b, 50, 64, 40, F16, out_dtype=F16)
    part = orc.matmul(a, b, 50, 64, 40, F16, out_dtype=F16, row0=17, nrows=9)
    assert np.array_equal(full[17:26], part)


# ---- causal mask ------------------------------------------------------------------------

def test_causal_mask_index_rule():
    x = np.arange(12 * 12, dtype=np.float32).reshape(12, 12)
    y = orc.causal_mask_f32(x, 12, 12)
    r, c = np.indices((12, 12))
    assert np.array_equal(y[c <= r], x[c <= r])
    assert (y.view(np.uint32)[c > r] == 0xFF800000).all()
    assert np.isneginf(y).sum() == 12 * 11 // 2


# ---- attention -------------------------------------------------------------------------------

def test_attention_f32_golden(golden):
    g = golden("attention_f32.npz")
    s, d = g["sd"]
    o = orc.attention_f32(g["q"], g["k"], g["v"], s, d)
    assert np.abs(o - g["o"]).max() < 2e-5


def test_attention_f32_uniform_keys_average_values():
    rng = np.random.default_rng(8)
    s, d = 40, 16
    q = rng.standard_normal((s, d)).astype(np.float32)
    k = np.tile(rng.standard_normal((1, d)).astype(np.float32), (s, 1))
    v = rng.standard_normal((s, d)).astype(np.float32)
    o = orc.attention_f32(q, k, v, s, d)
    assert np.allclose(o, np.tile(v.mean(axis=0), (s, 1)), atol=2e-6)


def _prefill_args(g):
    B, S, start, max_seq, D, NH, NKV = (int(t) for t in g["shape"])
    return B, S, start, max_seq, D, NH, NKV


def test_prefill_golden(golden):
    g = golden("prefill_bf16.npz")
    B, S, start, max_seq, D, NH, NKV = _prefill_args(g)
    o = orc.attention_prefill(g["q"], g["k"], g["v"], BF16, B, S, start, max_seq, D, NH, NKV)
    assert np.abs(o - g["o"].reshape(-1)).max() < 2e-5


def test_prefill_first_row_is_first_value():
    rng = np.random.default_rng(9)
    B, S, NH, NKV, D = 1, 8, 2, 1, 32
    q = orc.narrow(rng.standard_normal(B * S * NH * D).astype(np.float32), BF16)
    k = orc.narrow(rng.standard_normal(B * NKV * S * D).astype(np.float32), BF16)
    v = orc.narrow(rng.standard_normal(B * NKV * S * D).astype(np.float32), BF16)
    o = orc.attention_prefill(q, k, v, BF16, B, S, 0, S, D, NH, NKV).reshape(B, S, NH, D)
    v0 = orc.widen(v, BF16).reshape(B, NKV, S, D)[0, 0, 0]
    assert np.array_equal(o[0, 0, 0], v0) and np.array_equal(o[0, 0, 1], v0)


def test_prefill_gqa_equals_mha_with_repeated_kv():
    rng = np.random.default_rng(10)
    B, S, NH, NKV, D = 2, 20, 4, 2, 16
    q = orc.narrow(rng.standard_normal(B * S * NH * D).astype(np.float32), BF16)
    k = orc.narrow(rng.standard_normal(B * NKV * S * D).astype(np.float32), BF16)
    v = orc.narrow(rng.standard_normal(B * NKV * S * D).astype(np.float32), BF16)
    o_gqa = orc.attention_prefill(q, k, v, BF16, B, S, 0, S, D, NH, NKV)
    rep = lambda t: np.repeat(t.reshape(B, NKV, S, D), NH // NKV, axis=1).copy()
    o_mha = orc.attention_prefill(q, rep(k), rep(v), BF16, B, S, 0, S, D, NH, NH)
    assert np.array_equal(o_gqa, o_mha)


def test_decode_golden(golden):
    g = golden("decode_bf16.npz")
    B, L, max_seq, D, NH, NKV = (int(t) for t in g["shape"])
    o = orc.attention_decode(g["q"], g["k"], g["v"], BF16, B, L, max_seq, D, NH, NKV)
    assert np.abs(o - g["o"].reshape(-1)).max() < 2e-5


def test_decode_equals_last_prefill_row():
    rng = np.random.default_rng(11)
    B, NH, NKV, D, L, max_seq = 2, 4, 2, 32, 50, 64
    q = orc.narrow(rng.standard_normal(B * NH * D).astype(np.float32), BF16)
    k = orc.narrow(rng.standard_normal(B * NKV * max_seq * D).astype(np.float32), BF16)
    v = orc.narrow(rng.standard_normal(B * NKV * max_seq * D).astype(np.float32), BF16)
    od = orc.attention_decode(q, k, v, BF16, B, L, max_seq, D, NH, NKV)
    # one prefill query at absolute position L-1 sees positions 0..L-1
    op = orc.attention_prefill(q, k, v, BF16, B, 1, L - 1, max_seq, D, NH, NKV)
    assert np.array_equal(od, op)


def test_decode_single_position_returns_value():
    rng = np.random.default_rng(12)
    B, NH, NKV, D, max_seq = 1, 4, 1, 16, 8
    q = orc.narrow(rng.standard_normal(B * NH * D).astype(np.float32), BF16)
    k = orc.narrow(rng.standard_normal(B * NKV * max_seq * D).astype(np.float32), BF16)
    v = orc.narrow(rng.standard_normal(B * NKV * max_seq * D).astype(np.float32), BF16)
    o = orc.attention_decode(q, k, v, BF16, B, 1, max_seq, D, NH, NKV).reshape(NH, D)
    v0 = orc.widen(v, BF16)[:D]
    assert all(np.array_equal(o[h], v0) for h in range(NH))


# ---- elementwise, row reductions, transpose, matvec -----------------------------------------

def _ulps(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


def test_unary_closed_forms():
    e = np.float32(np.e)
    assert orc.unary_f32("exp", np.float32([0.0]))[0] == 1.0
    assert orc.unary_f32("log", np.float32([1.0]))[0] == 0.0
    assert _ulps(orc.unary_f32("log", np.float32([e, e * e])), [1.0, 2.0]).max() <= 1
    assert orc.unary_f32("sqrt", np.float32([4.0, 0.25]))[:].tolist() == [2.0, 0.5]
    assert orc.unary_f32("rsqrt", np.float32([4.0, 0.25]))[:].tolist() == [0.5, 2.0]
    assert orc.unary_f32("sigmoid", np.float32([0.0]))[0] == 0.5
    assert orc.unary_f32("tanh", np.float32([0.0]))[0] == 0.0
    assert orc.unary_f32("abs", np.float32([-3.5, 2.0])).tolist() == [3.5, 2.0]
    x = np.float32([-2.0, -0.0, 0.0, 1.5])
    assert orc.unary_f32("relu", x).tolist() == [0.0, 0.0, 0.0, 1.5]
    assert orc.unary_f32("neg", x).tolist() == [2.0, 0.0, -0.0, -1.5]


def test_unary_properties_and_numpy():
    rng = np.random.default_rng(21)
    x = (rng.standard_normal(4096) * 3).astype(np.float32)
    # odd / complementary functions
    assert np.array_equal(orc.unary_f32("tanh", -x), -orc.unary_f32("tanh", x))
    s, sm = orc.unary_f32("sigmoid", x), orc.unary_f32("sigmoid", -x)
    assert np.abs(s.astype(np.float64) + sm - 1.0).max() < 1.2e-7
    p = np.abs(x) + np.float32(1e-3)
    assert np.abs(orc.unary_f32("sqrt", p).astype(np.float64) ** 2 / p - 1).max() < 3e-7
    x64 = x.astype(np.float64)
    p64 = p.astype(np.float64)
    for op, ref in (("exp", np.exp(x64)), ("tanh", np.tanh(x64)), ("abs", np.abs(x64)),
                    ("sigmoid", 1.0 / (np.exp(-x64) + 1.0)), ("relu", np.maximum(x64, 0.0))):
        assert _ulps(orc.unary_f32(op, x), ref.astype(np.float32)).max() <= 1, op
    for op, ref in (("log", np.log(p64)), ("sqrt", np.sqrt(p64)), ("rsqrt", 1.0 / np.sqrt(p64))):
        assert _ulps(orc.unary_f32(op, p), ref.astype(np.float32)).max() <= 1, op


def test_minmax_exact():
    rng = np.random.default_rng(22)
    a, b = (rng.standard_normal(1000).astype(np.float32) for _ in range(2))
    b[::7] = a[::7]
    assert np.array_equal(orc.minmax_f32("min", a, b), np.minimum(a, b))
    assert np.array_equal(orc.minmax_f32("max", a, b), np.maximum(a, b))


def test_maximumf_minimumf_nan_and_signed_zero():
    """relu, min, max, clamp and the max reductions follow arith.maximumf / minimumf
    (IEEE 754-2019 maximum / minimum): NaN propagates, -0 < +0.  numpy's maximum and
    minimum propagate NaN too; the signed-zero rule is checked bit by bit."""
    rng = np.random.default_rng(25)
    a, b = (rng.standard_normal(1000).astype(np.float32) for _ in range(2))
    a[::13] = np.nan
    b[6::19] = np.nan
    got_max, got_min = orc.minmax_f32("max", a, b), orc.minmax_f32("min", a, b)
    assert np.array_equal(np.isnan(got_max), np.isnan(np.maximum(a, b)))
    assert np.array_equal(np.isnan(got_min), np.isnan(np.minimum(a, b)))
    ok = ~np.isnan(got_max)
    assert np.array_equal(got_max[ok], np.maximum(a, b)[ok])
    assert np.array_equal(got_min[ok], np.minimum(a, b)[ok])
    z = np.float32([-0.0, 0.0, -0.0, 0.0])
    w = np.float32([0.0, -0.0, -0.0, 0.0])
    assert np.signbit(orc.minmax_f32("max", z, w)).tolist() == [False, False, True, False]
    assert np.signbit(orc.minmax_f32("min", z, w)).tolist() == [True, True, True, False]
    r = orc.unary_f32("relu", np.float32([-0.0, np.nan, -1.0, 2.0]))
    assert not np.signbit(r[0]) and np.isnan(r[1]) and r[2] == 0.0 and r[3] == 2.0
    c = orc.clamp_f32(np.float32([np.nan, -3.0, 0.1, 9.0, -0.0]), -0.5, 0.75)
    assert np.isnan(c[0]) and c[1:4].tolist() == [-0.5, np.float32(0.1), 0.75] and np.signbit(c[4])
    x = rng.standard_normal((4, 50)).astype(np.float32)
    x[1, 30] = np.nan
    x[3, :] = -0.0
    x[3, 7] = 0.0
    m = orc.reduce_rows_f32("max", x, 4, 50)
    assert np.isnan(m[1]) and not np.isnan(m[[0, 2]]).any() and m[3] == 0 and not np.signbit(m[3])
    assert np.isnan(orc.reduce_rows_f32("absmax", x, 4, 50)[1])


def test_reduce_rows():
    rng = np.random.default_rng(23)
    R, C = 37, 301
    xi = rng.integers(-50, 50, (R, C)).astype(np.float32)  # integer sums are exact
    assert np.array_equal(orc.reduce_rows_f32("sum", xi, R, C), xi.sum(axis=1))
    x = rng.standard_normal((R, C)).astype(np.float32)
    assert np.array_equal(orc.reduce_rows_f32("max", x, R, C), x.max(axis=1))
    assert np.array_equal(orc.reduce_rows_f32("absmax", x, R, C), np.abs(x).max(axis=1))
    assert np.array_equal(orc.reduce_rows_f32("sum", x, R, C),
                          x.astype(np.float64).sum(axis=1).astype(np.float32))
    # argmax: first index of the maximum (ties planted), 0 when nothing exceeds -inf
    x[3, 10] = x[3, 200] = 50.0
    x[5, :] = -np.inf
    got = orc.reduce_rows_f32("argmax", x, R, C)
    assert got.dtype == np.int32 and got[3] == 10 and got[5] == 0
    assert np.array_equal(got, np.argmax(x, axis=1).astype(np.int32))


def test_transpose_and_matvec():
    rng = np.random.default_rng(24)
    R, C = 33, 70
    x = rng.standard_normal((R, C)).astype(np.float32)
    t = orc.transpose_f32(x, R, C).reshape(C, R)
    assert np.array_equal(t, x.T)
    assert np.array_equal(orc.transpose_f32(t, C, R).reshape(R, C), x)
    a = rng.integers(-20, 20, (R, C)).astype(np.float32)
    v = rng.integers(-20, 20, C).astype(np.float32)
    assert np.array_equal(orc.matvec_f32(a, v, R, C), (a.astype(np.int64) @ v.astype(np.int64)).astype(np.float32))
    e = np.zeros(C, np.float32)
    e[17] = 1.0
    assert np.array_equal(orc.matvec_f32(x, e, R, C), x[:, 17])  # picks one column

"""Parity tolerances for each tile op (HIP result vs the CPU oracle).

  softmax f32           |y - ref| <= 1e-5 * |ref| + 1e-30       (relative 1e-5)
  softmax f16 / bf16    at most one unit in the last place of the 16-bit format
  matmul (f32 out)      |c - ref| <= 1e-2 * |ref| + 1e-4 * rms(ref)
  matmul (16-bit out)   the same bound, with one 16-bit ulp of ref added
  attention (16-bit)    |o - ref| <= 2e-2 * |ref| + 1e-3  ... see ATTN_* below
  index / shape work    bit-exact (causal mask, integer-valued GEMM inputs)

The GEMM bound is "1e-2 relative"; the rms term keeps it meaningful for
entries near zero produced by cancellation (their absolute error scales with
the row/column norms, not with the entry).
"""
from __future__ import annotations

import numpy as np

SOFTMAX_RTOL = 1e-5
GEMM_RTOL = 1e-2
GEMM_ATOL_RMS = 1e-4
ATTN_RTOL = 2e-2
ATTN_ATOL = 1e-3


def _report(name, bad, got, ref, err):
    idx = np.argwhere(bad)[:5]
    flat = np.flatnonzero(bad)[:5]
    return (f"{name}: {int(bad.sum())} of {bad.size} elements out of tolerance; first at "
            f"{idx.tolist()}: got {got.reshape(-1)[flat]}, ref {ref.reshape(-1)[flat]}, "
            f"max err {float(err.max()):.3e}")


def assert_softmax_close(got: np.ndarray, ref: np.ndarray, name: str = "softmax"):
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    err = np.abs(got - ref)
    bad = err > SOFTMAX_RTOL * np.abs(ref) + 1e-30
    assert not bad.any(), _report(name, bad, got, ref, err)


def ulp16(ref_f32: np.ndarray, dtype: int) -> np.ndarray:
    """Spacing of the 16-bit format at |ref| (dtype 1 = f16, 2 = bf16)."""
    a = np.abs(ref_f32.astype(np.float64))
    mant = 10 if dtype == 1 else 7
    min_exp = -14 if dtype == 1 else -126
    e = np.floor(np.log2(np.maximum(a, 2.0 ** min_exp)))
    return 2.0 ** (e - mant)


def assert_within_ulp16(got_f32, ref_f32, dtype: int, ulps: float = 1.0, name: str = "u16"):
    got = got_f32.astype(np.float64)
    ref = ref_f32.astype(np.float64)
    err = np.abs(got - ref)
    bad = err > ulps * ulp16(ref, dtype) * (1 + 1e-12)
    assert not bad.any(), _report(name, bad, got, ref, err)


def assert_gemm_close(got, ref, name: str = "matmul", u16_dtype: int | None = None):
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    tol = GEMM_RTOL * np.abs(ref) + GEMM_ATOL_RMS * rms
    if u16_dtype is not None:
        tol = tol + ulp16(ref, u16_dtype)
    err = np.abs(got - ref)
    bad = err > tol
    assert not bad.any(), _report(name, bad, got, ref, err)


def assert_attn_close(got, ref, name: str = "attention", rtol: float = ATTN_RTOL,
                      atol: float = ATTN_ATOL):
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    err = np.abs(got - ref)
    bad = err > rtol * np.abs(ref) + atol
    assert not bad.any(), _report(name, bad, got, ref, err)

"""ctypes loader for the CPU oracle (oracle/liboracle.so) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module, and only as the checker (or the timed CPU baseline).  The product path
never does.  Every function restates the reference semantics cited in
oracle/oracle.c.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

F32, F16, BF16 = 0, 1, 2
_lib = None


def build() -> Path:
    subprocess.run(["make", "-B", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        vp, i64, i = C.c_void_p, C.c_int64, C.c_int
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_widen.argtypes = [vp, vp, i64, i]
        L.orc_narrow.argtypes = [vp, vp, i64, i]
        L.orc_num_threads.restype = i
        L.orc_softmax_f32.argtypes = [vp, vp, i64, i64]
        L.orc_softmax_u16.argtypes = [vp, vp, i64, i64, i]
        L.orc_matmul_rows.argtypes = [vp, vp, vp, i64, i64, i64, i, i, i, i, i64, i64]
        L.orc_matmul.argtypes = [vp, vp, vp, i64, i64, i64, i, i, i, i]
        L.orc_causal_mask_f32.argtypes = [vp, vp, i64, i64]
        L.orc_unary_f32.argtypes = [i, vp, vp, i64]
        L.orc_minmax_f32.argtypes = [i, vp, vp, vp, i64]
        L.orc_clamp_f32.argtypes = [vp, vp, i64, C.c_float, C.c_float]
        L.orc_reduce_rows_f32.argtypes = [i, vp, vp, i64, i64]
        L.orc_transpose_f32.argtypes = [vp, vp, i64, i64]
        L.orc_matvec_f32.argtypes = [vp, vp, vp, i64, i64]
        L.orc_rms_norm.argtypes = [vp, vp, i64, i64, C.c_double, i]
        L.orc_silu_mul.argtypes = [vp, vp, vp, i64, i]
        L.orc_rope.argtypes = [vp, vp, i64, i64, i64, i]
        L.orc_matmul_silu_mul_rows.argtypes = [vp, vp, vp, vp, i64, i64, i64, i, i, i, i64, i64]
        L.orc_attention_f32.argtypes = [vp, vp, vp, vp, i64, i64]
        L.orc_attention_prefill.argtypes = [vp, vp, vp, vp, i, i] + [i64] * 11
        L.orc_attention_decode.argtypes = [vp, vp, vp, vp, i, i] + [i64] * 8
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _dt_of(a: np.ndarray, dtype: int | None) -> int:
    if dtype is not None:
        return dtype
    return F32 if a.dtype == np.float32 else BF16


def num_threads() -> int:
    return lib().orc_num_threads()


# ---- conversions -------------------------------------------------------------------

def widen(a: np.ndarray, dtype: int) -> np.ndarray:
    a = np.ascontiguousarray(a)
    out = np.empty(a.shape, np.float32)
    lib().orc_widen(_ptr(a), _ptr(out), a.size, dtype)
    return out


def narrow(a: np.ndarray, dtype: int) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    if dtype == F32:
        return a.copy()
    out = np.empty(a.shape, np.uint16)
    lib().orc_narrow(_ptr(a), _ptr(out), a.size, dtype)
    return out


# ---- ops ------------------------------------------------------------------------------

def softmax(x: np.ndarray, rows: int, cols: int, dtype: int = F32) -> np.ndarray:
    x = np.ascontiguousarray(x)
    y = np.empty_like(x)
    if dtype == F32:
        lib().orc_softmax_f32(_ptr(x), _ptr(y), rows, cols)
    else:
        lib().orc_softmax_u16(_ptr(x), _ptr(y), rows, cols, dtype)
    return y


def matmul(a, b, m, k, n, in_dtype, out_dtype=F32, b_trans=False, row0=0, nrows=None):
    """C rows [row0, row0+nrows) of A*B (or A*B^T).  Returns (nrows, n)."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    nrows = m - row0 if nrows is None else nrows
    c = np.empty((nrows, n), np.float32 if out_dtype == F32 else np.uint16)
    lib().orc_matmul_rows(_ptr(a), _ptr(b), _ptr(c), m, k, n, in_dtype, in_dtype, out_dtype,
                          int(b_trans), row0, nrows)
    return c


def rms_norm(x: np.ndarray, rows: int, cols: int, eps: float, dtype: int = F32) -> np.ndarray:
    """y = x * rsqrt(sum(x^2)/cols + eps) per row (mlir_to_linalg.rs:1666-1763)."""
    x = np.ascontiguousarray(x)
    y = np.empty_like(x)
    lib().orc_rms_norm(_ptr(x), _ptr(y), rows, cols, float(eps), dtype)
    return y


def rope(x: np.ndarray, rows: int, cols: int, pos: int, dtype: int = F32) -> np.ndarray:
    """Rotary embedding of interleaved pairs at position pos (mlir_to_gpu.rs:1508-1557)."""
    x = np.ascontiguousarray(x)
    assert cols % 2 == 0
    y = np.empty_like(x)
    lib().orc_rope(_ptr(x), _ptr(y), rows, cols, pos, dtype)
    return y


def silu_mul(gate: np.ndarray, up: np.ndarray, dtype: int = F32) -> np.ndarray:
    """silu(gate) * up elementwise (mlir_to_linalg.rs:774-782, :425)."""
    gate = np.ascontiguousarray(gate)
    up = np.ascontiguousarray(up)
    assert gate.shape == up.shape and gate.dtype == up.dtype
    out = np.empty_like(gate)
    lib().orc_silu_mul(_ptr(gate), _ptr(up), _ptr(out), gate.size, dtype)
    return out


def matmul_silu_mul(a, b, up, m, k, n, in_dtype, out_dtype=F32, b_trans=False, row0=0,
                    nrows=None):
    """Rows [row0, row0+nrows) of silu(A*B) * UP; UP is the full m x n tensor."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    up = np.ascontiguousarray(up)
    nrows = m - row0 if nrows is None else nrows
    c = np.empty((nrows, n), np.float32 if out_dtype == F32 else np.uint16)
    lib().orc_matmul_silu_mul_rows(_ptr(a), _ptr(b), _ptr(up), _ptr(c), m, k, n, in_dtype,
                                   out_dtype, int(b_trans), row0, nrows)
    return c


def causal_mask_f32(x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_causal_mask_f32(_ptr(x), _ptr(y), rows, cols)
    return y


UNARY = {"exp": 0, "log": 1, "tanh": 2, "abs": 3, "sqrt": 4, "rsqrt": 5, "sigmoid": 6, "relu": 7,
         "neg": 8}
ROW_REDUCE = {"sum": 0, "max": 1, "absmax": 2, "argmax": 3}


def unary_f32(op: str, x: np.ndarray) -> np.ndarray:
    """Elementwise f32 op of the linalg bridge (oracle.c orc_unary_f32)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_unary_f32(UNARY[op], _ptr(x), _ptr(y), x.size)
    return y


def minmax_f32(op: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    y = np.empty_like(a)
    lib().orc_minmax_f32(1 if op == "max" else 0, _ptr(a), _ptr(b), _ptr(y), a.size)
    return y


def clamp_f32(x: np.ndarray, lo: float, hi: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_clamp_f32(_ptr(x), _ptr(y), x.size, lo, hi)
    return y


def reduce_rows_f32(op: str, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Row sum / max / absmax (f32) or argmax (int32) of a rows x cols tensor."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.int32 if op == "argmax" else np.float32)
    lib().orc_reduce_rows_f32(ROW_REDUCE[op], _ptr(x), _ptr(y), rows, cols)
    return y


def transpose_f32(x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows * cols, np.float32)
    lib().orc_transpose_f32(_ptr(x), _ptr(y), rows, cols)
    return y


def matvec_f32(a: np.ndarray, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    lib().orc_matvec_f32(_ptr(a), _ptr(x), _ptr(y), rows, cols)
    return y


def attention_f32(q, k, v, s, d) -> np.ndarray:
    q, k, v = (np.ascontiguousarray(t, np.float32) for t in (q, k, v))
    o = np.empty((s, d), np.float32)
    lib().orc_attention_f32(_ptr(q), _ptr(k), _ptr(v), _ptr(o), s, d)
    return o


def attention_prefill(q, k, v, dtype, batch, seq_len, start_pos, max_seq, head_dim, nh, nkv,
                      out_dtype=F32, bh0=0, nbh=None, q0=0, nq=None) -> np.ndarray:
    """Output has the full [B][S][NH][D] shape; only the selected (bh, q) are written."""
    q, k, v = (np.ascontiguousarray(t) for t in (q, k, v))
    nbh = batch * nh - bh0 if nbh is None else nbh
    nq = seq_len - q0 if nq is None else nq
    o = np.zeros(batch * seq_len * nh * head_dim, np.float32 if out_dtype == F32 else np.uint16)
    lib().orc_attention_prefill(_ptr(q), _ptr(k), _ptr(v), _ptr(o), dtype, out_dtype, batch,
                                seq_len, start_pos, max_seq, head_dim, nh, nkv, bh0, nbh, q0, nq)
    return o


def attention_decode(q, k, v, dtype, batch, seq_len, max_seq, head_dim, nh, nkv, out_dtype=F32,
                     bh0=0, nbh=None) -> np.ndarray:
    q, k, v = (np.ascontiguousarray(t) for t in (q, k, v))
    nbh = batch * nh - bh0 if nbh is None else nbh
    o = np.zeros(batch * nh * head_dim, np.float32 if out_dtype == F32 else np.uint16)
    lib().orc_attention_decode(_ptr(q), _ptr(k), _ptr(v), _ptr(o), dtype, out_dtype, batch,
                               seq_len, max_seq, head_dim, nh, nkv, bh0, nbh)
    return o

/*
 * CPU ORACLE — TEST INFRASTRUCTURE ONLY.
 *
 * This file is the parity checker for the HIP hot path, not part of it.  Only
 * `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`
 * may load it.  The product library (tile-rs_amd/csrc) never links or calls it.
 *
 * It restates, in plain C (OpenMP for the large cases), the numeric meaning that
 * tile-rs gives its tile ops.  The reference has no executable numeric path for
 * them: its `linalg` bridge only prints MLIR text, and the prefill/decode
 * semantics exist only as Metal template text.  Each function below cites the
 * reference lines it follows.
 *
 * Pinning (how each function is checked independently of this file):
 *   bf16/f16 conversions  — exhaustive 65536-pattern round trips, IEEE special
 *                            values, and numpy's float16 rounding for f16.
 *   softmax               — golden vectors from torch CPU, row sums = 1,
 *                            shift invariance, constant rows -> 1/C.
 *   matmul                — bit-exact brute force on small integer-valued
 *                            inputs, identity/permutation matrices, golden
 *                            vectors from torch CPU.
 *   causal mask           — exact index rule col <= row, -inf above.
 *   attention (f32)       — golden vectors from torch CPU; uniform-K -> mean(V).
 *   attention prefill     — golden vectors from torch CPU
 *                            scaled_dot_product_attention(is_causal=True), GQA
 *                            with NKV = NH reducing to MHA, row 0 -> V[0].
 *   attention decode      — equals the last row of prefill; one position -> V;
 *                            golden vectors from torch CPU.
 *   rms_norm              — golden vectors from torch CPU (F.rms_norm); scale
 *                            invariance at eps = 0; constant and one-hot rows;
 *                            mean(y^2) = mean / (mean + eps).
 *   silu_mul, matmul_silu_mul — golden vectors from torch CPU (F.silu);
 *                            silu(0) = 0, silu(x) - silu(-x) = x, silu(x) -> x
 *                            for large x; the matmul part as matmul.
 *   rope                  — pos = 0 is the identity; each pair keeps its
 *                            norm; unit pairs (1,0) and (0,1) land on
 *                            (cos t, sin t) and (-sin t, cos t) with t from a
 *                            float64 closed form; rope(rope(x, a), b) =
 *                            rope(x, a + b).
 * Nothing here is "parity unpinned".
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_EXPORT __attribute__((visibility("default")))

/* dtype codes shared with the product ABI (include/tilers_hip.h TH_DTYPE_*). */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2 };

/* ------------------------------------------------------------------------ */
/* 16-bit float conversions.                                                 */
/* The linalg bridge narrows with `arith.truncf` and widens with `arith.extf` */
/* (mlir_to_linalg.rs:1249-1303, :520-529): round-to-nearest-even narrowing  */
/* and exact widening.  bf16 shares the u16 carrier with f16                 */
/* (tile_std/src/lib.rs:182).                                                */
/* ------------------------------------------------------------------------ */

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

ORC_EXPORT float orc_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

ORC_EXPORT uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
        return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN, keep sign */
    }
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

ORC_EXPORT float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0x1fu) return bits_f32(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return bits_f32(sign);
        /* subnormal: man * 2^-24 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

ORC_EXPORT uint16_t orc_f32_to_f16(float f) {
    uint32_t u = f32_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) { /* inf or nan */
        return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
    }
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
    if (a < 0x38800000u) {
        /* result is subnormal (or zero): value / 2^-24, rounded to nearest even */
        float v = bits_f32(a) * 16777216.0f; /* exact scale by 2^24 */
        /* v < 1024; round half to even via the float's own rounding */
        float r = nearbyintf(v);
        return (uint16_t)(sign | (uint16_t)r);
    }
    uint32_t exp = ((a >> 23) - 112u) << 10;
    uint32_t man = (a >> 13) & 0x3ffu;
    uint32_t rest = a & 0x1fffu;
    uint32_t h = exp | man;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

static inline float load_elem(const void* p, int64_t i, int dtype) {
    switch (dtype) {
    case ORC_F16: return orc_f16_to_f32(((const uint16_t*)p)[i]);
    case ORC_BF16: return orc_bf16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
    }
}

static inline void store_elem(void* p, int64_t i, int dtype, float v) {
    switch (dtype) {
    case ORC_F16: ((uint16_t*)p)[i] = orc_f32_to_f16(v); break;
    case ORC_BF16: ((uint16_t*)p)[i] = orc_f32_to_bf16(v); break;
    default: ((float*)p)[i] = v; break;
    }
}

ORC_EXPORT void orc_widen(const void* src, float* dst, int64_t n, int dtype) {
    #pragma omp parallel for schedule(static) if (n > (1 << 16))
    for (int64_t i = 0; i < n; ++i) dst[i] = load_elem(src, i, dtype);
}

ORC_EXPORT void orc_narrow(const float* src, void* dst, int64_t n, int dtype) {
    #pragma omp parallel for schedule(static) if (n > (1 << 16))
    for (int64_t i = 0; i < n; ++i) store_elem(dst, i, dtype, src[i]);
}

ORC_EXPORT int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* Row softmax: `linalg.softmax dimension(1)` (mlir_to_linalg.rs:1305-1343).  */
/* Per row: m = max_j x_j; e_j = exp(x_j - m); s = sum_j e_j; y_j = e_j / s.  */
/* f32 arithmetic; the sum is carried in double and rounded once, which is   */
/* the exact value of the f32 sum up to its final rounding.                   */
/* ------------------------------------------------------------------------ */

static void softmax_row(const float* x, float* y, int64_t cols) {
    float m = -INFINITY;
    for (int64_t j = 0; j < cols; ++j) m = x[j] > m ? x[j] : m;
    double s = 0.0;
    for (int64_t j = 0; j < cols; ++j) {
        float e = expf(x[j] - m);
        y[j] = e;
        s += (double)e;
    }
    float sf = (float)s;
    for (int64_t j = 0; j < cols; ++j) y[j] = y[j] / sf;
}

ORC_EXPORT void orc_softmax_f32(const float* x, float* y, int64_t rows, int64_t cols) {
    #pragma omp parallel for schedule(static) if (rows * cols > (1 << 15))
    for (int64_t r = 0; r < rows; ++r) softmax_row(x + r * cols, y + r * cols, cols);
}

/* f16 / bf16 softmax (tile.rs:2163, :2912): widen exactly, f32 softmax, RNE back. */
ORC_EXPORT void orc_softmax_u16(const uint16_t* x, uint16_t* y, int64_t rows, int64_t cols,
                                int dtype) {
    #pragma omp parallel for schedule(static) if (rows * cols > (1 << 15))
    for (int64_t r = 0; r < rows; ++r) {
        float* buf = (float*)malloc(sizeof(float) * 2 * (size_t)cols);
        for (int64_t j = 0; j < cols; ++j) buf[j] = load_elem(x, r * cols + j, dtype);
        softmax_row(buf, buf + cols, cols);
        for (int64_t j = 0; j < cols; ++j) store_elem(y, r * cols + j, dtype, buf[cols + j]);
        free(buf);
    }
}

/* ------------------------------------------------------------------------ */
/* RMSNorm (__tile_rms_norm_f32(dst, src, eps, rows, cols), tile.rs:2063;    */
/* linalg mlir_to_linalg.rs:1666-1763): sq = x*x; red = sum over dim 1;      */
/* mean = red / cols; var = mean + eps; rs = rsqrt(var); y = x * rs.  The     */
/* sum is taken in double here (the f32 reduction order of a linalg lowering */
/* is unspecified); 16-bit I/O is widened exactly and narrowed RNE.          */
/* ------------------------------------------------------------------------ */

ORC_EXPORT void orc_rms_norm(const void* x, void* y, int64_t rows, int64_t cols, double eps,
                             int dtype) {
    #pragma omp parallel for schedule(static) if (rows * cols > (1 << 15))
    for (int64_t r = 0; r < rows; ++r) {
        double ss = 0.0;
        for (int64_t j = 0; j < cols; ++j) {
            double v = (double)load_elem(x, r * cols + j, dtype);
            ss += v * v;
        }
        double rs = 1.0 / sqrt(ss / (double)cols + eps);
        for (int64_t j = 0; j < cols; ++j)
            store_elem(y, r * cols + j, dtype,
                       (float)((double)load_elem(x, r * cols + j, dtype) * rs));
    }
}

/* RoPE (__tile_rope_f32(dst, src, pos, rows, cols), tile.rs:232, :2425; gpu  */
/* lowering mlir_to_gpu.rs:1508-1557, SPIR-V body mlir_to_spirv.rs:1418-1432): */
/* each row's interleaved pairs (x[2i], x[2i+1]) rotate by the angle           */
/* pos * freq_i, freq_i = 1 / 10000^(2i / cols).  Both lowerings form freq and */
/* the angle in f32, so this does too; the rotation is evaluated in double and */
/* narrowed once.                                                              */
ORC_EXPORT void orc_rope(const void* x, void* y, int64_t rows, int64_t cols, int64_t pos,
                         int dtype) {
    #pragma omp parallel for schedule(static) if (rows * cols > (1 << 15))
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = 0; i < cols / 2; ++i) {
            const float freq = 1.0f / powf(10000.0f, 2.0f * (float)i / (float)cols);
            const float ang = (float)pos * freq;
            const double c = cos((double)ang), s = sin((double)ang);
            const double e = (double)load_elem(x, r * cols + 2 * i, dtype);
            const double o = (double)load_elem(x, r * cols + 2 * i + 1, dtype);
            store_elem(y, r * cols + 2 * i, dtype, (float)(e * c - o * s));
            store_elem(y, r * cols + 2 * i + 1, dtype, (float)(e * s + o * c));
        }
}

/* SiLU * Mul (linalg mlir_to_linalg.rs:774-782: silu(x) = x / (1 + exp(-x)),  */
/* then the elementwise linalg.mul of :425): out = silu(gate) * up, double     */
/* math on exactly widened inputs, one RNE narrowing.                          */
static float silu_mul1(double g, double u) { return (float)(g / (1.0 + exp(-g)) * u); }

ORC_EXPORT void orc_silu_mul(const void* gate, const void* up, void* out, int64_t n, int dtype) {
    #pragma omp parallel for schedule(static) if (n > (1 << 15))
    for (int64_t i = 0; i < n; ++i)
        store_elem(out, i, dtype,
                   silu_mul1((double)load_elem(gate, i, dtype), (double)load_elem(up, i, dtype)));
}

/* ------------------------------------------------------------------------ */
/* Matmul: `linalg.fill 0` + `linalg.matmul` on f32 tensors                  */
/* (mlir_to_linalg.rs:1345-1393).  16-bit operands are widened exactly      */
/* (`arith.extf`) before the contraction, the accumulator is f32, and the    */
/* result is narrowed once with RNE when the output tile is f16/bf16         */
/* (tile.rs:2593 returns a u16 tile; tile.rs:2666 returns the f32 tile).     */
/* `b_trans` selects C = A * B^T with B stored N x K (tile.rs:2028, :2694).   */
/*                                                                          */
/* rows [row0, row0 + nrows) of C are produced; callers use row subsets to   */
/* keep full-size checks affordable.                                        */
/* ------------------------------------------------------------------------ */

ORC_EXPORT void orc_matmul_rows(const void* a, const void* b, void* c, int64_t m, int64_t k,
                                int64_t n, int a_dtype, int b_dtype, int c_dtype, int b_trans,
                                int64_t row0, int64_t nrows) {
    (void)m;
    /* Widen B once into an f32 K x N panel (transposing when B is N x K). */
    float* bw = (float*)malloc(sizeof(float) * (size_t)k * (size_t)n);
    #pragma omp parallel for schedule(static)
    for (int64_t kk = 0; kk < k; ++kk) {
        for (int64_t j = 0; j < n; ++j) {
            int64_t idx = b_trans ? j * k + kk : kk * n + j;
            bw[kk * n + j] = load_elem(b, idx, b_dtype);
        }
    }
    #pragma omp parallel
    {
        float* arow = (float*)malloc(sizeof(float) * (size_t)k);
        float* acc = (float*)malloc(sizeof(float) * (size_t)n);
        #pragma omp for schedule(dynamic, 1)
        for (int64_t r = row0; r < row0 + nrows; ++r) {
            for (int64_t kk = 0; kk < k; ++kk) arow[kk] = load_elem(a, r * k + kk, a_dtype);
            for (int64_t j = 0; j < n; ++j) acc[j] = 0.0f;
            for (int64_t kk = 0; kk < k; ++kk) {
                const float av = arow[kk];
                const float* brow = bw + kk * n;
                #pragma omp simd
                for (int64_t j = 0; j < n; ++j) acc[j] = fmaf(av, brow[j], acc[j]);
            }
            for (int64_t j = 0; j < n; ++j) store_elem(c, (r - row0) * n + j, c_dtype, acc[j]);
        }
        free(arow);
        free(acc);
    }
    free(bw);
}

ORC_EXPORT void orc_matmul(const void* a, const void* b, void* c, int64_t m, int64_t k, int64_t n,
                           int a_dtype, int b_dtype, int c_dtype, int b_trans) {
    orc_matmul_rows(a, b, c, m, k, n, a_dtype, b_dtype, c_dtype, b_trans, 0, m);
}

/* ------------------------------------------------------------------------ */
/* Causal mask (mlir_to_linalg.rs:1191-1247): keep x[r][c] when c <= r,     */
/* otherwise write -inf (0xFF800000).                                        */
/* ------------------------------------------------------------------------ */

/* C = silu(A.B) * UP for rows [row0, row0 + nrows): the matmul above with an */
/* f32 result (no intermediate rounding), then silu*mul with UP (c_dtype,     */
/* C's layout) and one RNE narrowing to c_dtype.                              */
ORC_EXPORT void orc_matmul_silu_mul_rows(const void* a, const void* b, const void* up, void* c,
                                         int64_t m, int64_t k, int64_t n, int ab_dtype,
                                         int c_dtype, int b_trans, int64_t row0, int64_t nrows) {
    float* acc = (float*)malloc(sizeof(float) * (size_t)nrows * (size_t)n);
    orc_matmul_rows(a, b, acc, m, k, n, ab_dtype, ab_dtype, ORC_F32, b_trans, row0, nrows);
    #pragma omp parallel for schedule(static) if (nrows * n > (1 << 15))
    for (int64_t i = 0; i < nrows * n; ++i)
        store_elem(c, i, c_dtype,
                   silu_mul1((double)acc[i], (double)load_elem(up, row0 * n + i, c_dtype)));
    free(acc);
}

ORC_EXPORT void orc_causal_mask_f32(const float* x, float* y, int64_t rows, int64_t cols) {
    const float ninf = bits_f32(0xff800000u);
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c) y[r * cols + c] = (c <= r) ? x[r * cols + c] : ninf;
}

/* ------------------------------------------------------------------------ */
/* Elementwise f32 ops of the linalg bridge (op table mlir_to_linalg.rs:     */
/* 423-455): min/max = linalg.min/max; exp, log, tanh, abs, sqrt = the named */
/* linalg/math ops; rsqrt = math.rsqrt; sigmoid = 1 / (exp(-x) + 1) and      */
/* relu = maximumf(x, 0) (generic bodies :762-789).  Each value is computed   */
/* in double from the f32 input and rounded once to f32.                    */
/* ------------------------------------------------------------------------ */
enum { ORC_EXP = 0, ORC_LOG, ORC_TANH, ORC_ABS, ORC_SQRT, ORC_RSQRT, ORC_SIGMOID, ORC_RELU,
       ORC_NEG };

/* arith.maximumf / arith.minimumf (the float body of linalg.max / linalg.min and of */
/* the relu, clamp and max-reduce generics): IEEE 754-2019 maximum / minimum.  A NaN */
/* operand gives NaN; -0 orders below +0; otherwise the larger (smaller) value.      */
static float maximumf(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a == b) return signbit(a) ? b : a; /* equal values, or +0 against -0 */
    return a > b ? a : b;
}
static float minimumf(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a == b) return signbit(a) ? a : b;
    return a < b ? a : b;
}

static double unary1(int op, double x) {
    switch (op) {
        case ORC_EXP: return exp(x);
        case ORC_LOG: return log(x);
        case ORC_TANH: return tanh(x);
        case ORC_ABS: return fabs(x);
        case ORC_SQRT: return sqrt(x);
        case ORC_RSQRT: return 1.0 / sqrt(x);
        case ORC_SIGMOID: return 1.0 / (exp(-x) + 1.0);
        case ORC_RELU: return (double)maximumf((float)x, 0.0f); /* maximumf(%in, 0.0) */
        default: return -x;
    }
}

ORC_EXPORT void orc_unary_f32(int op, const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = (float)unary1(op, (double)x[i]);
}

/* op 0 = min (linalg.min -> minimumf), 1 = max (linalg.max -> maximumf); exact in f32 */
ORC_EXPORT void orc_minmax_f32(int op, const float* a, const float* b, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = op ? maximumf(a[i], b[i]) : minimumf(a[i], b[i]);
}

/* clamp (mlir_to_linalg.rs:906-955): minimumf(maximumf(x, lo), hi) */
ORC_EXPORT void orc_clamp_f32(const float* x, float* y, int64_t n, float lo, float hi) {
    for (int64_t i = 0; i < n; ++i) y[i] = minimumf(maximumf(x[i], lo), hi);
}

/* ------------------------------------------------------------------------ */
/* Row reductions, dimension 1 of a rows x cols f32 tensor (mlir_to_linalg.rs:*/
/* 1496-1573): op 0 sum (init 0), 1 max (init -inf, combiner maximumf, so a  */
/* NaN in the row gives NaN), 2 absmax = the max reduce of linalg.abs(x).    */
/* The sum is carried in double and                                          */
/* rounded once.  op 3 argmax (:1576-1660): running (value, index) from      */
/* (-inf, 0), replaced when x > value (ordered compare), so the result is    */
/* the first index of the maximum and 0 for a row with no value above -inf.   */
/* argmax writes int32 indices into y's 32-bit slots.                        */
/* ------------------------------------------------------------------------ */
ORC_EXPORT void orc_reduce_rows_f32(int op, const float* x, void* y, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * cols;
        if (op == 0) {
            double s = 0.0;
            for (int64_t c = 0; c < cols; ++c) s += (double)xr[c];
            ((float*)y)[r] = (float)s;
        } else if (op == 3) {
            float v = bits_f32(0xff800000u);
            int32_t idx = 0;
            for (int64_t c = 0; c < cols; ++c)
                if (xr[c] > v) { v = xr[c]; idx = (int32_t)c; }
            ((int32_t*)y)[r] = idx;
        } else {
            float m = bits_f32(0xff800000u);
            for (int64_t c = 0; c < cols; ++c) m = maximumf(m, op == 2 ? fabsf(xr[c]) : xr[c]);
            ((float*)y)[r] = m;
        }
    }
}

/* Transpose (mlir_to_linalg.rs:1458-1490): rows x cols -> cols x rows. */
ORC_EXPORT void orc_transpose_f32(const float* x, float* y, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c) y[c * rows + r] = x[r * cols + c];
}

/* Matvec (mlir_to_linalg.rs:1395-1440): linalg.fill 0 + linalg.matvec,       */
/* y[r] = sum_c a[r][c] * x[c]; each sum carried in double, rounded once.   */
ORC_EXPORT void orc_matvec_f32(const float* a, const float* x, float* y, int64_t rows,
                               int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) {
        double s = 0.0;
        for (int64_t c = 0; c < cols; ++c) s += (double)a[r * cols + c] * (double)x[c];
        y[r] = (float)s;
    }
}

/* ------------------------------------------------------------------------ */
/* Single-head attention (mlir_to_linalg.rs:1781-1902):                     */
/*   Kt = transpose(K); S = Q * Kt; S *= (float)(1/sqrt(D)) computed in f64  */
/*   (:1843); P = softmax(S, dim 1); O = P * V.  Non-causal, f32.            */
/* ------------------------------------------------------------------------ */

ORC_EXPORT void orc_attention_f32(const float* q, const float* k, const float* v, float* o,
                                  int64_t s, int64_t d) {
    const float scale = (float)(1.0 / sqrt((double)d));
    #pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)s);
        float* p = (float*)malloc(sizeof(float) * (size_t)s);
        #pragma omp for schedule(static)
        for (int64_t i = 0; i < s; ++i) {
            for (int64_t j = 0; j < s; ++j) {
                float acc = 0.0f;
                for (int64_t t = 0; t < d; ++t) acc = fmaf(q[i * d + t], k[j * d + t], acc);
                row[j] = acc * scale;
            }
            softmax_row(row, p, s);
            for (int64_t t = 0; t < d; ++t) {
                float acc = 0.0f;
                for (int64_t j = 0; j < s; ++j) acc = fmaf(p[j], v[j * d + t], acc);
                o[i * d + t] = acc;
            }
        }
        free(row);
        free(p);
    }
}

/* ------------------------------------------------------------------------ */
/* Prefill attention, causal + GQA (mlir_to_msl.rs:10928-11009; host params */
/* :1851-1859).  For batch b, query position qi (absolute abs = start+qi),   */
/* head h:  kv_head = h / (NH / NKV); scale = rsqrt(D); keys at positions    */
/* pos <= abs of that kv head are scored, softmaxed and used to weight V.    */
/* Layouts: Q, O = [B][S][NH][D]; K, V = [B][NKV][max_seq][D].               */
/* The Metal template caps the KV length at 256 (:10943); the restatement    */
/* has no cap (the HIP kernels are flash kernels over the full length).       */
/* Inputs are widened exactly; all math is f32; O is narrowed with RNE.      */
/*                                                                          */
/* The (b, h) pairs and the query-row range to produce can be restricted:    */
/* heads are b*NH+h indices in [bh0, bh0+nbh); rows [q0, q0+nq).  The output */
/* buffer always has the full [B][S][NH][D] shape.                           */
/* ------------------------------------------------------------------------ */

ORC_EXPORT void orc_attention_prefill(const void* q, const void* k, const void* v, void* o,
                                      int dtype, int out_dtype, int64_t batch, int64_t seq_len,
                                      int64_t start_pos, int64_t max_seq, int64_t head_dim,
                                      int64_t nh, int64_t nkv, int64_t bh0, int64_t nbh,
                                      int64_t q0, int64_t nq) {
    (void)batch;
    const int64_t D = head_dim;
    const int64_t group = nh / nkv;
    const float scale = 1.0f / sqrtf((float)D);
    const int64_t total = nbh * nq;
    const int64_t L = start_pos + seq_len; /* positions any selected row can see */
    if (total <= 0 || L <= 0) return;
    /* The (b, kv_head) units the selected heads read, widened once: K transposed to   */
    /* [D][L] so that PB consecutive positions' dot products advance together (each    */
    /* one still a sequential fmaf chain over t = 0..D-1, the same operations in the   */
    /* same order as one dot at a time), V as [L][D].                                  */
    const int64_t u0 = (bh0 / nh) * nkv + (bh0 % nh) / group;
    const int64_t bl = bh0 + nbh - 1;
    const int64_t u1 = (bl / nh) * nkv + (bl % nh) / group + 1;
    const int64_t nu = u1 - u0;
    float* kt = (float*)malloc(sizeof(float) * (size_t)(nu * D * L));
    float* vf = (float*)malloc(sizeof(float) * (size_t)(nu * L * D));
    #pragma omp parallel for schedule(static) collapse(2)
    for (int64_t u = 0; u < nu; ++u)
        for (int64_t pos = 0; pos < L; ++pos) {
            const int64_t src = ((u0 + u) * max_seq + pos) * D;
            for (int64_t t = 0; t < D; ++t) {
                kt[(u * D + t) * L + pos] = load_elem(k, src + t, dtype);
                vf[(u * L + pos) * D + t] = load_elem(v, src + t, dtype);
            }
        }
    enum { PB = 16 };
    #pragma omp parallel
    {
        float* qv = (float*)malloc(sizeof(float) * (size_t)D);
        float* sc = (float*)malloc(sizeof(float) * (size_t)(L + PB));
        float* p = (float*)malloc(sizeof(float) * (size_t)L);
        float* acc = (float*)malloc(sizeof(float) * (size_t)D);
        #pragma omp for schedule(dynamic, 4)
        for (int64_t w = 0; w < total; ++w) {
            const int64_t bh = bh0 + w / nq;
            const int64_t qi = q0 + w % nq;
            const int64_t b = bh / nh, h = bh % nh;
            const int64_t kvh = h / group;
            const int64_t abs_pos = start_pos + qi;
            const int64_t q_off = ((b * seq_len + qi) * nh + h) * D;
            const int64_t u = b * nkv + kvh - u0;
            const float* ku = kt + u * D * L;
            const float* vu = vf + u * L * D;
            const int64_t n = abs_pos + 1; /* positions 0..abs_pos are unmasked */
            for (int64_t t = 0; t < D; ++t) qv[t] = load_elem(q, q_off + t, dtype);
            int64_t pos = 0;
            for (; pos + PB <= n; pos += PB) {
                float dot[PB];
                for (int j = 0; j < PB; ++j) dot[j] = 0.0f;
                for (int64_t t = 0; t < D; ++t) {
                    const float qt = qv[t];
                    const float* kr = ku + t * L + pos;
                    #pragma omp simd
                    for (int j = 0; j < PB; ++j) dot[j] = fmaf(qt, kr[j], dot[j]);
                }
                for (int j = 0; j < PB; ++j) sc[pos + j] = dot[j] * scale;
            }
            for (; pos < n; ++pos) {
                float dot = 0.0f;
                for (int64_t t = 0; t < D; ++t) dot = fmaf(qv[t], ku[t * L + pos], dot);
                sc[pos] = dot * scale;
            }
            softmax_row(sc, p, n);
            for (int64_t t = 0; t < D; ++t) acc[t] = 0.0f;
            for (int64_t ps = 0; ps < n; ++ps) {
                const float pp = p[ps];
                const float* vr = vu + ps * D;
                #pragma omp simd
                for (int64_t t = 0; t < D; ++t) acc[t] = fmaf(pp, vr[t], acc[t]);
            }
            for (int64_t t = 0; t < D; ++t) store_elem(o, q_off + t, out_dtype, acc[t]);
        }
        free(qv);
        free(sc);
        free(p);
        free(acc);
    }
    free(kt);
    free(vf);
}

/* ------------------------------------------------------------------------ */
/* Decode attention, GQA, one query token (mlir_to_msl.rs:10747-10816; host */
/* params :1816-1823).  For batch b and head h: kv_head = h / (NH / NKV);   */
/* scores over positions [0, seq_len) scaled by rsqrt(D); softmax; V sum.    */
/* Layouts: Q, O = [B][NH][D]; K, V = [B][NKV][max_seq][D].  No 256 cap.     */
/* ------------------------------------------------------------------------ */

ORC_EXPORT void orc_attention_decode(const void* q, const void* k, const void* v, void* o,
                                     int dtype, int out_dtype, int64_t batch, int64_t seq_len,
                                     int64_t max_seq, int64_t head_dim, int64_t nh, int64_t nkv,
                                     int64_t bh0, int64_t nbh) {
    (void)batch;
    const int64_t D = head_dim;
    const int64_t group = nh / nkv;
    const float scale = 1.0f / sqrtf((float)D);
    #pragma omp parallel
    {
        float* qv = (float*)malloc(sizeof(float) * (size_t)D);
        float* sc = (float*)malloc(sizeof(float) * (size_t)(seq_len > 0 ? seq_len : 1));
        float* p = (float*)malloc(sizeof(float) * (size_t)(seq_len > 0 ? seq_len : 1));
        float* acc = (float*)malloc(sizeof(float) * (size_t)D);
        #pragma omp for schedule(dynamic, 1)
        for (int64_t w = 0; w < nbh; ++w) {
            const int64_t bh = bh0 + w;
            const int64_t b = bh / nh, h = bh % nh;
            const int64_t kvh = h / group;
            const int64_t q_off = (b * nh + h) * D;
            const int64_t kv_base = (b * nkv + kvh) * max_seq * D;
            for (int64_t t = 0; t < D; ++t) qv[t] = load_elem(q, q_off + t, dtype);
            for (int64_t pos = 0; pos < seq_len; ++pos) {
                float dot = 0.0f;
                for (int64_t t = 0; t < D; ++t)
                    dot = fmaf(qv[t], load_elem(k, kv_base + pos * D + t, dtype), dot);
                sc[pos] = dot * scale;
            }
            softmax_row(sc, p, seq_len);
            for (int64_t t = 0; t < D; ++t) acc[t] = 0.0f;
            for (int64_t pos = 0; pos < seq_len; ++pos) {
                const float pp = p[pos];
                for (int64_t t = 0; t < D; ++t)
                    acc[t] = fmaf(pp, load_elem(v, kv_base + pos * D + t, dtype), acc[t]);
            }
            for (int64_t t = 0; t < D; ++t) store_elem(o, q_off + t, out_dtype, acc[t]);
        }
        free(qv);
        free(sc);
        free(p);
        free(acc);
    }
}

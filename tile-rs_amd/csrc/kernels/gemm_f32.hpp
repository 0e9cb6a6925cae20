// f32 GEMM on gfx950's fp32 matrix cores (v_mfma_f32_32x32x2_f32): the
// __tile_matmul_f32 op (crates/tile_std/src/tile.rs:193, :2309; linalg
// semantics crates/rustc_codegen_tile/src/mlir_to_linalg.rs:1345-1393: C = A.B
// with f32 accumulation).
//
// One 128 x 128 tile of C per 256-thread workgroup: 2 x 2 waves, each 64 x 64 =
// 2 x 2 blocks of 32 x 32 accumulators (64 registers).  K advances 16 at a time
// through two LDS buffers.  Both operands sit in LDS k-major, A^T[k][m] and
// B[k][n], because the MFMA's two k values per step go to the two lane halves
// (lane l holds A[m = l % 32][k = l / 32] and B[k = l / 32][n = l % 32]): every
// operand fetch is one 4-byte LDS read of 32 consecutive values per half.  Rows
// are 128 + 32 floats long so that rows k and k + 1 fall in opposite halves of
// the 64 banks.  A (and B^T when B is given as N x K) is transposed on its way
// into LDS; row-major B is copied as is.  The next K step's tiles are loaded
// into registers while the current one computes (one barrier per step).
//
// The MFMA multiplies and adds in f32 (no reduced-precision inputs); only the
// order of the K sum differs from a sequential FMA loop.
#pragma once

#include "common.hpp"
#include "gemm.hpp"

namespace th {
namespace gf32 {
constexpr int BM = 128, BN = 128, BK = 16;
// Tile-rows per XCD group.  Four workgroups per CU run an XCD's whole run of
// tiles at once (128 at 4096^3); groups 8 tall make that run 8 x 16 tiles, which
// reads 8 A and 16 B panels instead of 4 and 32 (groups 4 tall).
constexpr int GROUP_M = 8;
constexpr int LD = 128 + 32;  // LDS row (floats)
constexpr int NT = 256;

typedef float f32x16 __attribute__((ext_vector_type(16)));

// 16-byte aligned: row-major B tiles go in with 16-byte LDS writes
struct alignas(16) Lds {
  float a[2][BK * LD];
  float b[2][BK * LD];
};
__device__ __forceinline__ Lds& smem() {
  __shared__ Lds s;
  return s;
}

// 4 consecutive floats of row `r` (`cols` long, row stride `ld`) from column c,
// zero past the matrix; one 16-byte load when VEC and the 4 are in range.
template <bool VEC>
__device__ __forceinline__ f32x4 load4(const float* __restrict__ p, uint32_t r, uint32_t c,
                                       uint32_t rows, uint32_t cols, size_t ld) {
  f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
  if (r >= rows) return v;
  const float* q = p + static_cast<size_t>(r) * ld + c;
  if (VEC && c + 4 <= cols) return *reinterpret_cast<const f32x4*>(q);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (c + j < cols) v[j] = q[j];
  return v;
}
}  // namespace gf32

// Tile (tm, tn) of C (M x N, row stride N) = A (M x K) . B (K x N, or N x K when
// B_TRANS).  VEC: every row start of A and B is 16-byte aligned (K % 4 == 0 and,
// for row-major B, N % 4 == 0, aligned bases), so full 4-float pieces load as one.
template <int DT_OUT, bool B_TRANS, bool VEC, int EPI>
__device__ __forceinline__ void gemm_f32_tile_128(const float* __restrict__ A,
                                                  const float* __restrict__ B,
                                                  void* __restrict__ C, uint32_t M, uint32_t N,
                                                  uint32_t K, uint32_t tm, uint32_t tn,
                                                  const void* __restrict__ up) {
  using namespace gf32;
  Lds& s = smem();
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const uint32_t m0 = tm * BM, n0 = tn * BN;

  // staging: A piece i covers rows (t + 256 i) % 128, k (t + 256 i) / 128 * 4 ..+3,
  // so the 64 lanes of a wave write 64 consecutive m of one A^T row.
  constexpr int NP = BM * BK / 4 / NT;   // 16-byte pieces per thread per operand
  f32x4 ra[NP], rb[NP];
  auto load = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int e = t + 256 * i;
      ra[i] = load4<VEC>(A, m0 + (e & 127), k0 + (e >> 7) * 4, M, K, K);
      if constexpr (B_TRANS) rb[i] = load4<VEC>(B, n0 + (e & 127), k0 + (e >> 7) * 4, N, K, K);
      else rb[i] = load4<VEC>(B, k0 + (e >> 5), n0 + (e & 31) * 4, K, N, N);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int e = t + 256 * i;
      const int r = e & 127, k4 = (e >> 7) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) s.a[buf][(k4 + j) * LD + r] = ra[i][j];
      if constexpr (B_TRANS) {
#pragma unroll
        for (int j = 0; j < 4; ++j) s.b[buf][(k4 + j) * LD + r] = rb[i][j];
      } else {
        *reinterpret_cast<f32x4*>(&s.b[buf][(e >> 5) * LD + (e & 31) * 4]) = rb[i];
      }
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int h = lane >> 5, l32 = lane & 31;
  const int ao = wm * 64 + l32, bo = wn * 64 + l32;
  const uint32_t nk = (K + BK - 1) / BK;
  load(0);
  store(0);
  __syncthreads();
  for (uint32_t kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load((kt + 1) * BK);
    const float* sa = s.a[cur] + h * LD + ao;
    const float* sb = s.b[cur] + h * LD + bo;
#pragma unroll
    for (int ks = 0; ks < BK / 2; ++ks) {
      const float a0 = sa[2 * ks * LD], a1 = sa[2 * ks * LD + 32];
      const float b0 = sb[2 * ks * LD], b1 = sb[2 * ks * LD + 32];
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
    }
    if (kt + 1 < nk) store(cur ^ 1);
    __syncthreads();
  }

  // accumulator r of a 32 x 32 block: row 8 (r / 4) + 4 h + r % 4, column l32
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t col = n0 + wn * 64 + 32 * j + l32;
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t row = m0 + wm * 64 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
        if (row < M)
          gemm::store_out<EPI, DT_OUT>(C, up, static_cast<size_t>(row) * N + col, acc[i][j][r]);
      }
    }
}

// Library kernel: tiles in XCD-aware grouped order (GROUP_M), batch = blockIdx.y with
// element strides sa, sb, sc.
template <int DT_OUT, bool B_TRANS, bool VEC, int EPI = 0>
__global__ void __launch_bounds__(gf32::NT)
gemm_f32_mfma(const float* __restrict__ A, const float* __restrict__ B, void* __restrict__ C,
              uint32_t M, uint32_t N, uint32_t K, uint64_t sa, uint64_t sb, uint64_t sc,
              const void* __restrict__ up) {
  constexpr int OSZ = (DT_OUT == kF32) ? 4 : 2;
  const uint32_t tiles_m = (M + gf32::BM - 1) / gf32::BM, tiles_n = (N + gf32::BN - 1) / gf32::BN;
  uint32_t tm, tn;
  gemm::tile_coords<gf32::GROUP_M>(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const size_t co = static_cast<size_t>(blockIdx.y) * sc * OSZ;
  gemm_f32_tile_128<DT_OUT, B_TRANS, VEC, EPI>(
      A + blockIdx.y * sa, B + blockIdx.y * sb, static_cast<char*>(C) + co, M, N, K, tm, tn,
      up ? static_cast<const char*>(up) + co : nullptr);
}

}  // namespace th

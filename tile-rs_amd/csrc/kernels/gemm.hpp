// Dense GEMM C[M,N] = A[M,K] * B[K,N] (or B stored N x K, `B_TRANS`).
//
// Semantics: `linalg.fill 0` + `linalg.matmul` with f32 accumulation
// (reference: crates/rustc_codegen_tile/src/mlir_to_linalg.rs:1345-1393).
// Intrinsics: __tile_matmul_f16 (crates/tile_std/src/tile.rs:1983) with the
// u16-tile result (tile.rs:2593) or the f32-tile result (`_acc_f32`,
// tile.rs:2666); __tile_matmul_transposed_f16 (tile.rs:2028, :2694);
// __tile_matmul_f32 (tile.rs:193, :2309) uses the f32 fallback kernel below.
//
// MFMA path (gfx950): 256x256 macro-tile per workgroup, K staged 64 at a time
// through LDS with two buffers, four waves each owning a 128x128 sub-tile of
// 4x4 v_mfma_f32_32x32x16_{bf16,f16} accumulators (f32).  Global tiles are
// fetched into registers one K-step ahead, so the HBM/L2 latency of step k+1
// hides behind the MFMAs of step k.  In LDS both operands are stored with K
// contiguous (row = 64 elements = 128 B = 8 chunks of 16 B) and the 16-byte chunk
// index is XOR-swizzled by the row so that 8 consecutive lanes always touch 8
// different chunks (conflict-free 128-bit reads and writes).  A row-major B is
// transposed 8x8 in registers on its way into LDS.
//
// The 1-D hardware grid is mapped to tiles XCD-first: workgroups are dealt to
// the 8 XCDs round-robin, so hardware block b is renumbered so that each XCD
// receives a contiguous run of tile ids, and runs are laid out GROUP_M tile-rows
// tall; tiles that share A rows or B columns then share one XCD's L2.
#pragma once

#include "common.hpp"

namespace th {

namespace gemm {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int NT = 256;          // threads per workgroup
constexpr int GROUP_M = 4;       // tile-rows per swizzle group
constexpr int NXCD = 8;          // XCDs on MI355X

__device__ __forceinline__ int swz(int row, int chunk) {
  return chunk ^ ((row ^ (row >> 3)) & 7);
}

// Map hardware block id -> (tile_m, tile_n).
__device__ __forceinline__ void tile_coords(uint32_t bid, uint32_t tiles_m, uint32_t tiles_n,
                                            uint32_t& tm, uint32_t& tn) {
  const uint32_t total = tiles_m * tiles_n;
  uint32_t id = bid;
  if (total % NXCD == 0) id = (bid % NXCD) * (total / NXCD) + bid / NXCD;
  const uint32_t per_group = GROUP_M * tiles_n;
  const uint32_t group = id / per_group;
  const uint32_t first_m = group * GROUP_M;
  const uint32_t gm = min(tiles_m - first_m, static_cast<uint32_t>(GROUP_M));
  const uint32_t in_group = id % per_group;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

}  // namespace gemm

// One 256x256 output tile (tm, tn) of C = A*B by a whole workgroup.
template <int DT, int DT_OUT, bool B_TRANS>
__device__ __forceinline__ void gemm_tile_256(const uint16_t* __restrict__ A,
                                              const uint16_t* __restrict__ B,
                                              void* __restrict__ C, uint32_t M, uint32_t N,
                                              uint32_t K, uint32_t tm, uint32_t tn) {
  using namespace gemm;
  __shared__ u32x4 lds_a[2][BM * BK / 8];
  __shared__ u32x4 lds_b[2][BN * BK / 8];
  const uint32_t m0 = tm * BM, n0 = tn * BN;

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l32 = lane & 31, g = lane >> 5;

  u32x4 ra[8], rb[8];

  auto load_tile = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = t + NT * i;
      const int row = c >> 3, kc = c & 7;
      const uint32_t gm_ = m0 + row, gk = k0 + kc * 8;
      ra[i] = (gm_ < M && gk < K) ? ldg128(A + static_cast<size_t>(gm_) * K + gk) : u32x4{0, 0, 0, 0};
    }
    if constexpr (B_TRANS) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int c = t + NT * i;
        const int row = c >> 3, kc = c & 7;
        const uint32_t gn = n0 + row, gk = k0 + kc * 8;
        rb[i] = (gn < N && gk < K) ? ldg128(B + static_cast<size_t>(gn) * K + gk) : u32x4{0, 0, 0, 0};
      }
    } else {
      const int kb = t >> 5, nb = t & 31;
      const uint32_t gn = n0 + nb * 8;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const uint32_t gk = k0 + kb * 8 + r;
        rb[r] = (gn < N && gk < K) ? ldg128(B + static_cast<size_t>(gk) * N + gn) : u32x4{0, 0, 0, 0};
      }
    }
  };

  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = t + NT * i;
      const int row = c >> 3, kc = c & 7;
      lds_a[buf][row * 8 + swz(row, kc)] = ra[i];
    }
    if constexpr (B_TRANS) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int c = t + NT * i;
        const int row = c >> 3, kc = c & 7;
        lds_b[buf][row * 8 + swz(row, kc)] = rb[i];
      }
    } else {
      const int kb = t >> 5, nb = t & 31;
      u32x4 tr[8];
      transpose8x8_b16(rb, tr);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int row = nb * 8 + j;
        lds_b[buf][row * 8 + swz(row, kb)] = tr[j];
      }
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const uint32_t nk = (K + BK - 1) / BK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (uint32_t kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tile((kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int chunk = 2 * ks + g;
      u32x4 fa[4], fb[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        const int row = wm * 128 + mi * 32 + l32;
        fa[mi] = lds_a[cur][row * 8 + swz(row, chunk)];
      }
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
        const int row = wn * 128 + ni * 32 + l32;
        fb[ni] = lds_b[cur][row * 8 + swz(row, chunk)];
      }
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma32x32x16<DT>(fa[mi], fb[ni], acc[mi][ni]);
    }
    if (kt + 1 < nk) store_tile(cur ^ 1);
    __syncthreads();
  }

  // Epilogue.  Accumulator register r of lane l in a 32x32 block holds
  // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      const uint32_t col = n0 + wn * 128 + ni * 32 + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t row = m0 + wm * 128 + mi * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (row < M && col < N) {
          const size_t off = static_cast<size_t>(row) * N + col;
          if constexpr (DT_OUT == kF32) {
            static_cast<float*>(C)[off] = acc[mi][ni][r];
          } else {
            static_cast<uint16_t*>(C)[off] = f32_to_u16<DT_OUT>(acc[mi][ni][r]);
          }
        }
      }
    }
}

// A: M x K (K contiguous).  B: K x N (N contiguous) or, with B_TRANS, N x K.
// Requires K % 8 == 0 and, for row-major B, N % 8 == 0; M, N, K tails are handled
// by zero-filled loads and predicated stores.  Batch index = blockIdx.y with
// element strides sa, sb, sc.
template <int DT, int DT_OUT, bool B_TRANS>
__global__ void __launch_bounds__(gemm::NT, 1)
gemm_mfma_256(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, void* __restrict__ C,
              uint32_t M, uint32_t N, uint32_t K, uint64_t sa, uint64_t sb, uint64_t sc) {
  const uint32_t tiles_m = (M + gemm::BM - 1) / gemm::BM, tiles_n = (N + gemm::BN - 1) / gemm::BN;
  uint32_t tm, tn;
  gemm::tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  constexpr int OSZ = (DT_OUT == kF32) ? 4 : 2;
  gemm_tile_256<DT, DT_OUT, B_TRANS>(A + blockIdx.y * sa, B + blockIdx.y * sb,
                                     static_cast<char*>(C) + blockIdx.y * sc * OSZ, M, N, K, tm, tn);
}

// Fallback for shapes the MFMA path does not take (K % 8 != 0, row-major B with
// N % 8 != 0) and for f32 operands: 64x64 tile per 256-thread workgroup, each
// thread a 4x4 block, K staged 16 at a time through LDS, f32 FMA.
template <int DT, int DT_OUT, bool B_TRANS>
__device__ __forceinline__ void gemm_fma_tile_64(const void* __restrict__ A,
                                                 const void* __restrict__ B, void* __restrict__ C,
                                                 uint32_t M, uint32_t N, uint32_t K, uint32_t tile) {
  __shared__ float as[16][64 + 4];
  __shared__ float bs[16][64 + 4];
  const uint32_t m0 = tile / ((N + 63) / 64) * 64;
  const uint32_t n0 = tile % ((N + 63) / 64) * 64;
  const int t = threadIdx.x;
  const int tr = t / 16, tc = t % 16;
  float acc[4][4] = {};
  auto ld = [&](const void* p, size_t i) -> float {
    if constexpr (DT == kF32) return static_cast<const float*>(p)[i];
    else return u16_to_f32<DT>(static_cast<const uint16_t*>(p)[i]);
  };
  const size_t boffA = 0, boffB = 0;
  for (uint32_t k0 = 0; k0 < K; k0 += 16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = t + 256 * i;  // 1024 elements per 64x16 panel
      const int r = e / 16, kk = e % 16;
      const uint32_t gm_ = m0 + r, gk = k0 + kk;
      as[kk][r] = (gm_ < M && gk < K) ? ld(A, boffA + static_cast<size_t>(gm_) * K + gk) : 0.0f;
      const uint32_t gn = n0 + r;
      float bv = 0.0f;
      if (gn < N && gk < K) {
        bv = B_TRANS ? ld(B, boffB + static_cast<size_t>(gn) * K + gk)
                     : ld(B, boffB + static_cast<size_t>(gk) * N + gn);
      }
      bs[kk][r] = bv;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = as[kk][tr * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = bs[kk][tc * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t row = m0 + tr * 4 + i, col = n0 + tc * 4 + j;
      if (row < M && col < N) {
        const size_t off = static_cast<size_t>(row) * N + col;
        if constexpr (DT_OUT == kF32) static_cast<float*>(C)[off] = acc[i][j];
        else static_cast<uint16_t*>(C)[off] = f32_to_u16<DT_OUT>(acc[i][j]);
      }
    }
}

template <int DT, int DT_OUT, bool B_TRANS>
__global__ void __launch_bounds__(256)
gemm_fma_64(const void* __restrict__ A, const void* __restrict__ B, void* __restrict__ C,
            uint32_t M, uint32_t N, uint32_t K, uint64_t sa, uint64_t sb, uint64_t sc) {
  constexpr int ISZ = (DT == kF32) ? 4 : 2;
  constexpr int OSZ = (DT_OUT == kF32) ? 4 : 2;
  gemm_fma_tile_64<DT, DT_OUT, B_TRANS>(static_cast<const char*>(A) + blockIdx.y * sa * ISZ,
                                        static_cast<const char*>(B) + blockIdx.y * sb * ISZ,
                                        static_cast<char*>(C) + blockIdx.y * sc * OSZ, M, N, K,
                                        blockIdx.x);
}

}  // namespace th

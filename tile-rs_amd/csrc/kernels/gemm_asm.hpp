// Dense 16-bit GEMM on whole 256 x 256 tiles: the library's kernel for M and N multiples
// of 256 and K a multiple of 128 (at least 256), B row-major (K x N) or stored N x K
// (BT, __tile_matmul_transposed_f16: crates/tile_std/src/tile.rs:2028).
//
// The tile program is generated gfx950 assembly (gen_gemm.py, run by the build into
// kernels/gen/gemm_asm.inc): four waves of 128 x 128 with AGPR accumulators
// (v_mfma_f32_16x16x32), A fetched
// in 64-deep double stages (whole 128-byte rows per DMA lane group), B in 32-deep
// stages; layouts, schedule and waits are described in gen_gemm.py.  This wrapper maps
// the workgroup to its tile and computes the per-lane and per-wave operands.
// Semantics: C = A . B with f32 accumulation (crates/rustc_codegen_tile/src/
// mlir_to_linalg.rs:1345-1393), C rounded once (RNE) to its dtype; K runs in the same
// order as in gemm_dma_256, and both give the same bits (checked on both config shapes).
#pragma once

#include "gemm.hpp"
#include "kernels/gen/gemm_asm.inc"

namespace th {
namespace gasm {
constexpr int NT = 256;   // 4 waves
// Shapes the program takes: whole tiles, K in groups of four 32-deep steps (at least
// two groups), and every per-lane byte offset within 32 bits.
__host__ __device__ constexpr bool fits(uint64_t m, uint64_t n, uint64_t k, int out_size) {
  return m % 256 == 0 && n % 256 == 0 && k % 128 == 0 && k >= 256 && m > 0 && n > 0 &&
         256 * k * 2 < (1ull << 31) && 136 * n * out_size < (1ull << 31) && 32 * n * 2 < (1ull << 31);
}
}  // namespace gasm

// Tile (tm, tn) of C = A . B by a workgroup of gasm::NT threads (launched with at most
// one workgroup per CU: the program uses all 512 registers of each lane).  A, B
// 16-byte aligned, C aligned to its element; gasm::fits(M, N, K, sizeof C) holds.  A
// workgroup that runs several tiles passes a barrier between them (the next tile's
// DMA refills buffers the previous one's last reads used).
// SILU: C = silu(A . B) * UP (kEpiSiluMul), UP an M x N tensor of C's 16-bit dtype and
// layout, 16-byte aligned.
template <int DT, int DT_OUT, bool BT = false, bool SILU = false>
__device__ __forceinline__ void gemm_asm_tile(const uint16_t* __restrict__ A,
                                              const uint16_t* __restrict__ B,
                                              void* __restrict__ C, uint32_t M, uint32_t N,
                                              uint32_t K, uint32_t tm, uint32_t tn,
                                              const void* __restrict__ UP = nullptr) {
  static_assert(DT == kBF16 || DT == kF16, "16-bit operands");
  static_assert(!SILU || DT_OUT != kF32, "the SiLU*Mul program writes 16-bit C");
  constexpr uint32_t OSZ = (DT_OUT == kF32) ? 4 : 2;
  char* Cb = static_cast<char*>(C);
  u32x4* arena = lds::dma_lds_arena<131072>();
  typedef __attribute__((address_space(3))) const void* lds_cptr;
  const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_cptr)(arena)));
  const uint32_t m0 = tm * 256, n0 = tn * 256;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t wm = wave >> 1, wn = wave & 1;
  const uint64_t abase = reinterpret_cast<uint64_t>(A + static_cast<size_t>(m0) * K);
  const uint64_t bbase = reinterpret_cast<uint64_t>(BT ? B + static_cast<size_t>(n0) * K : B + n0);
  const uint64_t cbase = reinterpret_cast<uint64_t>(
      Cb + (static_cast<size_t>(m0 + wm * 128) * N + n0 + wn * 128) * OSZ);
  // A double stage [256 r][8 chunks]: chunk c of row r at c ^ (r & 7)
  auto swa = [](uint32_t r) { return r & 7; };
  // B stage [32 k][32 chunks]: chunk c of k-row r at c ^ sb(r)
  auto swb = [](uint32_t r) { return 4 * (r & 3) ^ 2 * ((r >> 3) & 1); };
  // DMA: A unit j of wave w = rows 64 w + 8 j + lane / 8, position lane % 8 (units 0
  // and 1 here; the program derives the others); B unit j = k rows 2 (4 w + j) +
  // lane / 32, position lane % 32 holding chunk (lane % 32) ^ sb(k).
  uint32_t aoff[2], boff[4], ra[2], rb[4];
#pragma unroll
  for (uint32_t j = 0; j < 2; ++j) {
    const uint32_t row = 64 * wave + 8 * j + lane / 8;
    aoff[j] = row * K * 2 + (((lane & 7) ^ swa(row)) << 4);
  }
  if constexpr (BT) {
    // B^T double stages: the same units and swizzle as A, over the tile's n rows
#pragma unroll
    for (uint32_t j = 0; j < 2; ++j) boff[j] = aoff[j];
    boff[2] = boff[3] = 0;
  } else {
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      const uint32_t kr = 2 * (4 * wave + j) + lane / 32;
      boff[j] = kr * N * 2 + (((lane & 31) ^ swb(kr)) << 4);
    }
  }
  // Fragment reads (16x16x32 operands).  A (k half h): lane reads row 128 wm + 16 mi +
  // lane % 16, chunk 4 h + lane / 16 (mi as an immediate: 2 KB per 16 rows).
#pragma unroll
  for (uint32_t h = 0; h < 2; ++h) {
    const uint32_t row = wm * 128 + (lane & 15);
    ra[h] = row * 128 + (((4 * h + (lane >> 4)) ^ swa(row)) << 4);
  }
  if constexpr (BT) {
    // B^T (k half h): lane reads n row 128 wn + 16 ni + lane % 16, chunk 4 h + lane / 16
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h) {
      const uint32_t row = wn * 128 + (lane & 15);
      rb[h] = row * 128 + (((4 * h + (lane >> 4)) ^ swa(row)) << 4);
    }
    rb[2] = rb[3] = 0;
  } else {
    // B^T from row-major B: lane (q, i) = (lane / 16, lane % 16) reads k rows 8 q +
    // (i >> 2) (+4 as an immediate: same sb) at column n = 128 wn + 16 ni + 4 (i & 3);
    // passed for the even blocks ni = 2p (the program flips chunk bit 1 for the odd ones).
    const uint32_t q = lane >> 4, i = lane & 15;
    const uint32_t k0 = 8 * q + (i >> 2);
#pragma unroll
    for (uint32_t p = 0; p < 4; ++p) {
      const uint32_t n = wn * 128 + 32 * p + 4 * (i & 3);
      rb[p] = k0 * 512 + (((n >> 3) ^ swb(k0)) << 4) + (n & 7) * 2;
    }
  }
  // C: after the epilogue's lane swap, lane l writes row 8 (l / 32), column l % 32 of
  // each row group and pair of column blocks
  const uint32_t coff = ((8 * (lane >> 5)) * N + (lane & 31)) * OSZ;
  const uint32_t nk = K / 32, bstep = 64 * N, nstride = N * OSZ, arow8 = 16 * K;
  const uint32_t ldsa = lds + wave * 8192, ldsb = lds + 65536 + wave * (BT ? 8192 : 4096);
  if constexpr (SILU) {
    // UP: the wave's 128 x 128 tile, staged row-major in the wave's 32 KB of the ring
    // (256-byte rows); DMA unit j = rows 4 j + lane / 16, chunk lane % 16.  Reads
    // follow the epilogue's lane swap: lane l takes row 8 (l / 32) (+ immediates),
    // column l % 32.
    const uint64_t ubase = reinterpret_cast<uint64_t>(
        static_cast<const char*>(UP) + (static_cast<size_t>(m0 + wm * 128) * N + n0 + wn * 128) * 2);
    const uint32_t ustage = lds + wave * 32768;
    const uint32_t uoff = (lane >> 4) * N * 2 + (lane & 15) * 16;
    const uint32_t uread = ustage + 2048 * (lane >> 5) + 2 * (lane & 31);
#define TH_GEMM_ASM_SILU_OPS(STR)                                                                \
  asm volatile(STR                                                                              \
               :                                                                                \
               : "v"(aoff[0]), "v"(aoff[1]), "v"(boff[0]), "v"(boff[1]), "v"(boff[2]),         \
                 "v"(boff[3]), "v"(ra[0]), "v"(ra[1]), "v"(rb[0]), "v"(rb[1]), "v"(rb[2]),      \
                 "v"(rb[3]), "v"(coff), "s"(abase), "s"(bbase),                                 \
                 "s"(cbase), "s"(nk), "s"(lds), "s"(ldsa), "s"(ldsb), "s"(bstep), "s"(nstride), \
                 "s"(arow8), "s"(ubase), "s"(ustage), "v"(uoff), "v"(uread)                     \
               : TH_GEMM_ASM_SILU_CLOBBERS, "vcc", "scc", "memory")
    if constexpr (BT) {
      if constexpr (DT == kBF16) {
        if constexpr (DT_OUT == kBF16) TH_GEMM_ASM_SILU_OPS(TH_GEMM_ASM_SILU_BF16_BF16_BT);
        else TH_GEMM_ASM_SILU_OPS(TH_GEMM_ASM_SILU_BF16_F16_BT);
      } else {
        if constexpr (DT_OUT == kBF16) TH_GEMM_ASM_SILU_OPS(TH_GEMM_ASM_SILU_F16_BF16_BT);
        else TH_GEMM_ASM_SILU_OPS(TH_GEMM_ASM_SILU_F16_F16_BT);
      }
    } else if constexpr (DT == kBF16) {
      if constexpr (DT_OUT == kBF16) TH_GEMM_ASM_SILU_OPS(TH_GEMM_ASM_SILU_BF16_BF16);
      else TH_GEMM_ASM_SILU_OPS(TH_GEMM_ASM_SILU_BF16_F16);
    } else {
      if constexpr (DT_OUT == kBF16) TH_GEMM_ASM_SILU_OPS(TH_GEMM_ASM_SILU_F16_BF16);
      else TH_GEMM_ASM_SILU_OPS(TH_GEMM_ASM_SILU_F16_F16);
    }
#undef TH_GEMM_ASM_SILU_OPS
    return;
  }
#define TH_GEMM_ASM_OPS(STR)                                                                    \
  asm volatile(STR                                                                              \
               :                                                                                \
               : "v"(aoff[0]), "v"(aoff[1]), "v"(boff[0]), "v"(boff[1]), "v"(boff[2]),         \
                 "v"(boff[3]), "v"(ra[0]), "v"(ra[1]), "v"(rb[0]), "v"(rb[1]), "v"(rb[2]),      \
                 "v"(rb[3]), "v"(coff), "s"(abase), "s"(bbase),                                 \
                 "s"(cbase), "s"(nk), "s"(lds), "s"(ldsa), "s"(ldsb), "s"(bstep), "s"(nstride), \
                 "s"(arow8)                                                                     \
               : TH_GEMM_ASM_CLOBBERS, "vcc", "scc", "memory")
  if constexpr (BT) {
    if constexpr (DT == kBF16) {
      if constexpr (DT_OUT == kF32) TH_GEMM_ASM_OPS(TH_GEMM_ASM_BF16_F32_BT);
      else if constexpr (DT_OUT == kBF16) TH_GEMM_ASM_OPS(TH_GEMM_ASM_BF16_BF16_BT);
      else TH_GEMM_ASM_OPS(TH_GEMM_ASM_BF16_F16_BT);
    } else {
      if constexpr (DT_OUT == kF32) TH_GEMM_ASM_OPS(TH_GEMM_ASM_F16_F32_BT);
      else if constexpr (DT_OUT == kBF16) TH_GEMM_ASM_OPS(TH_GEMM_ASM_F16_BF16_BT);
      else TH_GEMM_ASM_OPS(TH_GEMM_ASM_F16_F16_BT);
    }
  } else if constexpr (DT == kBF16) {
    if constexpr (DT_OUT == kF32) TH_GEMM_ASM_OPS(TH_GEMM_ASM_BF16_F32);
    else if constexpr (DT_OUT == kBF16) TH_GEMM_ASM_OPS(TH_GEMM_ASM_BF16_BF16);
    else TH_GEMM_ASM_OPS(TH_GEMM_ASM_BF16_F16);
  } else {
    if constexpr (DT_OUT == kF32) TH_GEMM_ASM_OPS(TH_GEMM_ASM_F16_F32);
    else if constexpr (DT_OUT == kBF16) TH_GEMM_ASM_OPS(TH_GEMM_ASM_F16_BF16);
    else TH_GEMM_ASM_OPS(TH_GEMM_ASM_F16_F16);
  }
#undef TH_GEMM_ASM_OPS
}

// Batch index = blockIdx.y (element strides sa, sb, sc; UP, with SILU, strides like C).
template <int DT, int DT_OUT, bool BT = false, bool SILU = false>
__global__ void __launch_bounds__(gasm::NT, 1)
gemm_asm_256(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, void* __restrict__ C,
             uint32_t M, uint32_t N, uint32_t K, uint64_t sa, uint64_t sb, uint64_t sc,
             const void* __restrict__ UP = nullptr) {
  constexpr uint32_t OSZ = (DT_OUT == kF32) ? 4 : 2;
  uint32_t tm, tn;
  gemm::tile_coords(blockIdx.x, M / 256, N / 256, tm, tn);
  const size_t coff = static_cast<size_t>(blockIdx.y) * sc * OSZ;
  gemm_asm_tile<DT, DT_OUT, BT, SILU>(A + blockIdx.y * sa, B + blockIdx.y * sb,
                                      static_cast<char*>(C) + coff, M, N, K, tm, tn,
                                      SILU ? static_cast<const char*>(UP) + coff : nullptr);
}
}  // namespace th

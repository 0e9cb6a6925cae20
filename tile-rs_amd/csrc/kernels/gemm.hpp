// Dense GEMM C[M,N] = A[M,K] * B[K,N] (or B stored N x K, `B_TRANS`).
//
// Semantics: `linalg.fill 0` + `linalg.matmul` with f32 accumulation
// (reference: crates/rustc_codegen_tile/src/mlir_to_linalg.rs:1345-1393).
// Intrinsics: __tile_matmul_f16 (crates/tile_std/src/tile.rs:1983) with the
// u16-tile result (tile.rs:2593) or the f32-tile result (`_acc_f32`,
// tile.rs:2666); __tile_matmul_transposed_f16 (tile.rs:2028, :2694).
// __tile_matmul_f32 (tile.rs:193, :2309) runs on the fp32 MFMA kernel of
// gemm_f32.hpp; the FMA kernel at the end of this file serves only 16-bit shapes
// the MFMA paths cannot take.
//
// Two MFMA paths (gfx950), both on 256x256 macro-tiles with
// v_mfma_f32_32x32x16_{bf16,f16} and f32 accumulators:
//  - gemm_dma_256 (the direct-to-LDS pipeline further down, ping-pong schedule)
//    for K a multiple of 32: the path every config shape takes;
//  - gemm_mfma_256, register-staged, for the other 16-bit shapes (K a multiple
//    of 8): K staged 64 at a time through LDS with two buffers, four waves each
//    owning a 128x128 sub-tile.  Global tiles are fetched into registers one
//    K-step ahead, so the HBM/L2 latency of step k+1 hides behind the MFMAs of
//    step k.  In LDS both operands are stored with K contiguous (row = 64
//    elements = 128 B = 8 chunks of 16 B) and the 16-byte chunk index is
//    XOR-swizzled by the row so that 8 consecutive lanes always touch 8
//    different chunks (conflict-free 128-bit reads and writes).  A row-major B
//    is transposed 8x8 in registers on its way into LDS.
//
// The 1-D hardware grid is mapped to tiles XCD-first: workgroups are dealt to
// the 8 XCDs round-robin, so hardware block b is renumbered so that each XCD
// receives a contiguous run of tile ids, and runs are laid out GROUP_M tile-rows
// tall; tiles that share A rows or B columns then share one XCD's L2.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace th {

namespace gemm {
// Output stage shared by the GEMM kernels.  kEpiStore: C = acc.  kEpiSiluMul:
// C = silu(acc) * UP, UP an M x N tensor of C's dtype and layout, with
// silu(x) = x / (1 + exp(-x)) (mlir_to_linalg.rs:774-782) and the product an
// elementwise mul (mlir_to_linalg.rs:425); computed in f32, rounded once.
enum : int { kEpiStore = 0, kEpiSiluMul = 1 };
template <int EPI, int DT_OUT>
__device__ __forceinline__ void store_out(void* __restrict__ C, const void* __restrict__ up,
                                          size_t off, float v) {
  if constexpr (EPI == kEpiSiluMul) {
    const float u = (DT_OUT == kF32) ? static_cast<const float*>(up)[off]
                                     : u16_to_f32<DT_OUT>(static_cast<const uint16_t*>(up)[off]);
    v = v / (1.0f + expf(-v)) * u;
  }
  // Nontemporal: C is not read again by this kernel (measured 1-4% faster than
  // ordinary stores for 4096^3 and 8192x4096x14336).
  if constexpr (DT_OUT == kF32) __builtin_nontemporal_store(v, static_cast<float*>(C) + off);
  else __builtin_nontemporal_store(f32_to_u16<DT_OUT>(v), static_cast<uint16_t*>(C) + off);
}

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int NT = 256;          // threads per workgroup
constexpr int GROUP_M = 4;       // tile-rows per swizzle group
constexpr int NXCD = 8;          // XCDs on MI355X

__device__ __forceinline__ int swz(int row, int chunk) {
  return chunk ^ ((row ^ (row >> 3)) & 7);
}

// Map hardware block id -> (tile_m, tile_n).  GM: tile-rows per group (an XCD's
// contiguous run of ids covers GM rows and run / GM columns of tiles).
template <int GM = GROUP_M>
__device__ __forceinline__ void tile_coords(uint32_t bid, uint32_t tiles_m, uint32_t tiles_n,
                                            uint32_t& tm, uint32_t& tn) {
  const uint32_t total = tiles_m * tiles_n;
  uint32_t id = bid;
  if (total % NXCD == 0) id = (bid % NXCD) * (total / NXCD) + bid / NXCD;
  const uint32_t per_group = GM * tiles_n;
  const uint32_t group = id / per_group;
  const uint32_t first_m = group * GM;
  const uint32_t gm = min(tiles_m - first_m, static_cast<uint32_t>(GM));
  const uint32_t in_group = id % per_group;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

// The workgroup's LDS for the MFMA GEMM: one allocation shared by every
// instantiation that is inlined into a kernel (2 stages of A and B, 128 KB).
struct GemmLds {
  u32x4 a[2][BM * BK / 8];
  u32x4 b[2][BN * BK / 8];
};
__device__ __forceinline__ GemmLds& gemm_lds() {
  __shared__ GemmLds lds;
  return lds;
}

}  // namespace gemm

// One 256x256 output tile (tm, tn) of C = A*B by a whole workgroup.
//
// Schedule per K-step of 64 (two LDS buffers, `cur` and `nxt`):
//   - MFMA fragments of sub-step ks+1 are read from LDS while the 16 MFMAs of
//     sub-step ks run (two register sets);
//   - the A and B tiles of step k+1, already in registers, are written to the
//     `nxt` buffer between sub-steps (nobody reads `nxt` in this step);
//   - after the step's barrier the global loads of step k+2 are issued, so they
//     have a whole step to land.
// FULL = M, N multiples of 256 and K of 64: no bounds checks in the loop.
template <int DT, int DT_OUT, bool B_TRANS, bool FULL, int WM = 2, int WN = 2, int EPI = 0>
__device__ __forceinline__ void gemm_tile_256(const uint16_t* __restrict__ A,
                                              const uint16_t* __restrict__ B,
                                              void* __restrict__ C, uint32_t M, uint32_t N,
                                              uint32_t K, uint32_t tm, uint32_t tn,
                                              const void* __restrict__ up = nullptr) {
  using namespace gemm;
  constexpr int NTH = 64 * WM * WN;     // threads in the workgroup
  constexpr int TM = BM / WM / 32;      // 32x32 accumulator blocks per wave, M
  constexpr int TN = BN / WN / 32;      // and N
  constexpr int LA = BM * BK / 8 / NTH; // 16-byte A chunks per thread per K-step
  GemmLds& lds = gemm_lds();
  auto& lds_a = lds.a;
  auto& lds_b = lds.b;
  const uint32_t m0 = tm * BM, n0 = tn * BN;

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, g = lane >> 5;

  // Staging.  With 256 threads every thread loads LA chunks of A and one 8x8
  // block (or 8 chunks) of B.  With 512 threads waves 0-3 load B and waves 4-7
  // load A, 8 chunks each, into one shared register array.
  constexpr bool SPLIT = NTH == 512;
  constexpr int NA = SPLIT ? 8 : LA;
  u32x4 ra[NA], rb_own[SPLIT ? 1 : 8];
  u32x4* rb = SPLIT ? ra : rb_own;
  const int ta = SPLIT ? t - 256 : t;   // index among the A loaders
  const int tb = t;                      // index among the B loaders (t < 256)
  const bool is_a = !SPLIT || t >= 256;
  const bool is_b = !SPLIT || t < 256;

  auto load_b = [&](uint32_t k0) {
    if constexpr (B_TRANS) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int c = tb + 256 * i;
        const int row = c >> 3, kc = c & 7;
        const uint32_t gn = n0 + row, gk = k0 + kc * 8;
        const uint16_t* p = B + static_cast<size_t>(gn) * K + gk;
        rb[i] = (FULL || (gn < N && gk < K)) ? ldg128(p) : u32x4{0, 0, 0, 0};
      }
    } else {
      const int kb = tb >> 5, nb = tb & 31;
      const uint32_t gn = n0 + nb * 8;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const uint32_t gk = k0 + kb * 8 + r;
        const uint16_t* p = B + static_cast<size_t>(gk) * N + gn;
        rb[r] = (FULL || (gn < N && gk < K)) ? ldg128(p) : u32x4{0, 0, 0, 0};
      }
    }
  };
  auto load_a = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int c = ta + 256 * i;
      const int row = c >> 3, kc = c & 7;
      const uint32_t gm_ = m0 + row, gk = k0 + kc * 8;
      const uint16_t* p = A + static_cast<size_t>(gm_) * K + gk;
      ra[i] = (FULL || (gm_ < M && gk < K)) ? ldg128(p) : u32x4{0, 0, 0, 0};
    }
  };
  auto load_tile = [&](uint32_t k0) {
    if constexpr (SPLIT) {
      if (is_a) load_a(k0);
      else load_b(k0);
    } else {
      load_a(k0);
      load_b(k0);
    }
  };

  auto store_a = [&](int buf) {
    if (is_a) {
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const int c = ta + 256 * i;
        const int row = c >> 3, kc = c & 7;
        lds_a[buf][row * 8 + swz(row, kc)] = ra[i];
      }
    }
  };
  auto store_b = [&](int buf) {
    if (is_b) {
      if constexpr (B_TRANS) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int c = tb + 256 * i;
          const int row = c >> 3, kc = c & 7;
          lds_b[buf][row * 8 + swz(row, kc)] = rb[i];
        }
      } else {
        // 8x8 transpose in registers, one output column (4 dwords) at a time.
        const int kb = tb >> 5, nb = tb & 31;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int dw = j >> 1;
          u32x4 col;
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            const uint32_t lo = rb[2 * p][dw], hi = rb[2 * p + 1][dw];
            col[p] = (j & 1) ? pack_halves<true>(lo, hi) : pack_halves<false>(lo, hi);
          }
          const int row = nb * 8 + j;
          lds_b[buf][row * 8 + swz(row, kb)] = col;
        }
      }
    }
  };

  // Fragment register sets: two (read ks+1 during the MFMAs of ks) with one
  // wave per SIMD; one with two waves per SIMD, where the other wave hides the
  // LDS latency and the registers are needed for the accumulators.
  constexpr int FS = SPLIT ? 1 : 2;
  u32x4 fa[FS][TM], fb[FS][TN];
  auto load_frags = [&](int buf, int ks, int set) {
    const int chunk = 2 * ks + g;
#pragma unroll
    for (int mi = 0; mi < TM; ++mi) {
      const int row = wm * (BM / WM) + mi * 32 + l32;
      fa[set][mi] = lds_a[buf][row * 8 + swz(row, chunk)];
    }
#pragma unroll
    for (int ni = 0; ni < TN; ++ni) {
      const int row = wn * (BN / WN) + ni * 32 + l32;
      fb[set][ni] = lds_b[buf][row * 8 + swz(row, chunk)];
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const uint32_t nk = (K + BK - 1) / BK;
  load_tile(0);
  store_a(0);
  store_b(0);
  __syncthreads();
  if (nk > 1) load_tile(BK);
  load_frags(0, 0, 0);

  for (uint32_t kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1, nxt = cur ^ 1;
    const bool more = kt + 1 < nk;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int set = (FS == 2) ? (ks & 1) : 0;
      if (FS == 1 && ks > 0) load_frags(cur, ks, 0);
      if (FS == 2 && ks + 1 < BK / 16) load_frags(cur, ks + 1, set ^ 1);
#pragma unroll
      for (int mi = 0; mi < TM; ++mi)
#pragma unroll
        for (int ni = 0; ni < TN; ++ni)
          acc[mi][ni] = mfma32x32x16<DT>(fa[set][mi], fb[set][ni], acc[mi][ni]);
      if (ks == 1 && more) store_a(nxt);
      if (ks == 2 && more) store_b(nxt);
    }
    __syncthreads();
    if (more) {
      if (kt + 2 < nk) load_tile((kt + 2) * BK);
      load_frags(nxt, 0, 0);
    }
  }

  // Epilogue.  Accumulator register r of lane l in a 32x32 block holds
  // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
  for (int mi = 0; mi < TM; ++mi)
#pragma unroll
    for (int ni = 0; ni < TN; ++ni) {
      const uint32_t col = n0 + wn * (BN / WN) + ni * 32 + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t row = m0 + wm * (BM / WM) + mi * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (FULL || (row < M && col < N))
          store_out<EPI, DT_OUT>(C, up, static_cast<size_t>(row) * N + col, acc[mi][ni][r]);
      }
    }
}

// A: M x K (K contiguous).  B: K x N (N contiguous) or, with B_TRANS, N x K.
// Requires K % 8 == 0 and, for row-major B, N % 8 == 0; M, N, K tails are handled
// by zero-filled loads and predicated stores (FULL = no tails: M, N multiples of
// 256 and K of 64).  Batch index = blockIdx.y with element strides sa, sb, sc.
template <int DT, int DT_OUT, bool B_TRANS, int WM, int WN, bool FULL, int EPI = 0>
__global__ void __launch_bounds__(64 * WM * WN, 1)
gemm_mfma_256(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, void* __restrict__ C,
              uint32_t M, uint32_t N, uint32_t K, uint64_t sa, uint64_t sb, uint64_t sc,
              const void* __restrict__ up) {
  const uint32_t tiles_m = (M + gemm::BM - 1) / gemm::BM, tiles_n = (N + gemm::BN - 1) / gemm::BN;
  uint32_t tm, tn;
  gemm::tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  constexpr int OSZ = (DT_OUT == kF32) ? 4 : 2;
  const size_t co = static_cast<size_t>(blockIdx.y) * sc * OSZ;
  gemm_tile_256<DT, DT_OUT, B_TRANS, FULL, WM, WN, EPI>(
      A + blockIdx.y * sa, B + blockIdx.y * sb, static_cast<char*>(C) + co, M, N, K, tm, tn,
      up ? static_cast<const char*>(up) + co : nullptr);
}

// ---------------------------------------------------------------------------
// Direct-to-LDS pipeline (the path for K a multiple of 32; any M, N).
//
// 256x256 tile per workgroup, eight waves (two per SIMD) each owning a 128x64
// sub-tile of 4x2 v_mfma_f32_32x32x16 accumulators.  K is staged 32 at a time
// through a ring of NS LDS buffers (4 x 32 KB by default) filled by
// global_load_lds_dwordx4: each lane's 16 bytes go straight from L2/HBM into
// LDS (no registers, no ds_write).
//
// Ping-pong schedule.  Waves 0-3 (group 0, one per SIMD) own rows 0-127 and
// waves 4-7 (group 1) rows 128-255, so each SIMD holds one wave of each group.
// Every K step has two phases per wave, each closed by a workgroup barrier:
//   memory phase:  read the step's MFMA fragments (both 16-k sub-steps) from LDS
//                  and wait for them; wait for this wave's share of the next
//                  stage's DMA;
//   compute phase: refill the buffer every wave has finished reading with the
//                  stage NS-1 ahead, then issue the step's 16 MFMAs back to back.
// Group 1 starts one phase late (an extra barrier before its first step, group 0
// one after its last), so on every SIMD one wave's MFMA burst runs while the
// other wave does its LDS reads and DMA issue.  Against both waves interleaving
// reads and MFMAs with one barrier per step: 4096^3 bf16 118.9 -> 109.7 us on one
// box, bit-identical output.
//   A stage: [256 m][32 k], 64-byte rows; 16-byte chunk c of row r sits at
//            c ^ ((r >> 2) & 3) -> conflict-free 128-bit MFMA reads.
//   B stage: row-major B needs no transpose anywhere: it stays [32 k][256 n]
//            (512-byte rows, chunk c at c ^ 4*(k & 3), so the four k rows one
//            half-wave reads land in four different 64-byte bank groups of the
//            64-bank LDS) and the MFMA B operand is read with
//            ds_read_b64_tr_b16, which hands each lane of a 16-lane group one
//            n column of a 4 (k) x 16 (n) block: two reads give the eight
//            consecutive k values of the 32x32x16 operand.
//   B_TRANS: B stage is [256 n][32 k] like A.
// The swizzles are applied on the global side: each lane picks the global
// chunk whose swizzled LDS slot is its own fixed slot (lane*16 bytes).
// ---------------------------------------------------------------------------
namespace gemm {
using lds::bar;
using lds::dma16;
using lds::dma_lds_arena;
using lds::lds_v4i16;
using lds::v4i16;
using lds::wait_vm;
constexpr int DBK = 32;       // K per stage (default shape)
constexpr int NSTAGE = 4;     // stages (default shape)
constexpr int DWAVES = 8;     // 2 x 4 waves of 128 x 64 (2 waves per SIMD)
// Wait until at most `later` stages of NL loads each are still in flight.
template <int NL, int MAXL>
__device__ __forceinline__ void wait_stages(uint32_t later) {
  if constexpr (MAXL >= 3) {
    if (later >= 3) { wait_vm<3 * NL>(); return; }
  }
  if constexpr (MAXL >= 2) {
    if (later >= 2) { wait_vm<2 * NL>(); return; }
  }
  if constexpr (MAXL >= 1) {
    if (later >= 1) { wait_vm<NL>(); return; }
  }
  wait_vm<0>();
}
}  // namespace gemm

// ldk: row stride along K of A (and of B when B_TRANS), 0 = K; a split-K caller
// passes the full K with K the slice depth.
// MI: 32-row blocks each wave computes (4 = its whole 128 rows).  Fewer serve
// tiles whose rows past 32 * MI (in each wave's half) are never stored: the
// small-M split-K launches, where most of a 256-row tile is padding.
template <int DT, int DT_OUT, bool B_TRANS, int KB = gemm::DBK, int NS = gemm::NSTAGE,
          int WAVES = gemm::DWAVES, int EPI = 0, int MI = 4>
__device__ __forceinline__ void gemm_dma_tile_256(const uint16_t* __restrict__ A,
                                                  const uint16_t* __restrict__ B,
                                                  void* __restrict__ C, uint32_t M, uint32_t N,
                                                  uint32_t K, uint32_t tm, uint32_t tn,
                                                  const void* __restrict__ up = nullptr,
                                                  uint32_t ldk = 0) {
  using namespace gemm;
  const size_t lk = ldk ? ldk : K;
  static_assert(KB == 32, "stage K: two 16-k sub-steps per step");
  static_assert(WAVES == 8, "ping-pong: two groups of one wave per SIMD");
  static_assert(NS >= 3, "a refill lands at least one step ahead of its use");
  static_assert(NS * (BM + BN) * KB * 2 <= 160 * 1024, "LDS");
  constexpr int NTH = 64 * WAVES;          // threads
  constexpr int WN_W = WAVES / 2;          // waves along N
  constexpr int TWN = BN / WN_W;           // wave tile N (128 or 64)
  constexpr int NI = TWN / 32;             // 32-wide MFMA blocks per wave along N
  constexpr int CPR = KB / 8;              // 16-byte chunks per A row
  constexpr int SA = BM * KB / 8;          // u32x4 per A stage
  constexpr int SB = BN * KB / 8;          // u32x4 per B stage
  constexpr int NLA = SA / NTH;            // DMA per thread per stage, A (and B)
  static_assert(NLA >= 1 && SA % NTH == 0, "stage split");
  u32x4* arena = dma_lds_arena<NS * (BM + BN) * KB * 2>();
  auto lds_a = [&](int st) { return arena + st * (SA + SB); };
  auto lds_b = [&](int st) { return arena + st * (SA + SB) + SA; };
  // A-like rows (k contiguous, CPR chunks): chunk c of row r at c ^ sw(r)
  auto swa = [](int row) { return CPR == 4 ? ((row >> 2) & 3) : ((row ^ (row >> 3)) & 7); };
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: SGPR LDS addresses
  const int wm = wave / WN_W, wn = wave % WN_W;
  const int l32 = lane & 31, g = lane >> 5;
  // A tile that crosses M or N reads a valid row (column chunk) in place of each
  // missing one; those values reach only outputs past M or N, which are not stored.
  const bool edge = m0 + BM > M || n0 + BN > N;

  // ---- per-thread DMA sources (NLA A chunks + NLA B chunks per stage) ----
  // Each wave-level load fills 1 KB of LDS (64 slots of 16 B); load j of wave w
  // fills slots (NLA*w + j)*64 ... Lane l owns slot l of that block.
  const uint16_t* srcA[NLA];
  const uint16_t* srcB[NLA];
#pragma unroll
  for (int j = 0; j < NLA; ++j) {
    const int slot = (NLA * wave + j) * 64 + lane;
    const int row = slot / CPR, c = (slot % CPR) ^ swa(row);
    srcA[j] = A + static_cast<size_t>(min(m0 + row, M - 1)) * lk + 8 * c;
    if constexpr (B_TRANS) {
      srcB[j] = B + static_cast<size_t>(min(n0 + row, N - 1)) * lk + 8 * c;
    } else {
      // [KB k][256 n] rows of 32 chunks; chunk c of k-row r at c ^ 4*(r & 3)
      const int kr = slot / 32, cb = (slot % 32) ^ (4 * (kr & 3));
      srcB[j] = B + static_cast<size_t>(kr) * N + min(n0 + 8 * cb, N - 8);
    }
  }
  auto issue = [&](uint32_t stage, uint32_t kt) {
    const size_t ka = static_cast<size_t>(kt) * KB;  // element offset along K
#pragma unroll
    for (int j = 0; j < NLA; ++j) dma16(srcA[j] + ka, lds_a(stage) + (NLA * wave + j) * 64);
#pragma unroll
    for (int j = 0; j < NLA; ++j) {
      const uint16_t* p = B_TRANS ? srcB[j] + ka : srcB[j] + ka * N;
      dma16(p, lds_b(stage) + (NLA * wave + j) * 64);
    }
  };

  // ---- fragment reads: a whole step (two 16-k sub-steps) per memory phase ----
  static_assert(MI == 1 || MI == 2 || MI == 4, "live row blocks");
  static_assert(EPI != kEpiSiluMul || MI == 4, "the staged epilogue covers whole tiles");
  static_assert(NI == 2, "two 32-column blocks per wave");
  constexpr int KS = KB / 16;
  u32x4 fa[KS][MI], fb[KS][NI];
  auto load_frags = [&](int stage) {
    const u32x4* la = lds_a(stage);
    const u32x4* lb = lds_b(stage);
    auto read_a = [&](int ks) {
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
        const int row = wm * 128 + mi * 32 + l32;
        fa[ks][mi] = la[row * CPR + ((2 * ks + g) ^ swa(row))];
      }
    };
    if constexpr (B_TRANS) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        read_a(ks);
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
          const int row = wn * TWN + ni * 32 + l32;
          fb[ks][ni] = lb[row * CPR + ((2 * ks + g) ^ swa(row))];
        }
      }
      lds::wait_lgkm0();
    } else {
      // Lane (q, i) of each 16-lane group reads k rows 16 ks + 8 (q >> 1) + 4 r + (i >> 2)
      // at column n = wn*64 + 32 ni + 16 (q & 1) + 4 (i & 3): one address per column
      // block, the (ks, r) steps as immediate offsets (16 ks + 4 r rows of 512 bytes).
      // The transposed reads are inline asm: the compiler would otherwise order them
      // after every outstanding LDS DMA (vmcnt(0)), which this schedule orders itself
      // with its stage waits and barriers.  One statement issues all eight and waits
      // for them, so no result is read (or copied) before it has landed.
      const int q = lane >> 4, i = lane & 15;
      const int k0 = 8 * (q >> 1) + (i >> 2);
      uint32_t addr[NI];
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        const int n = wn * TWN + ni * 32 + 16 * (q & 1) + 4 * (i & 3);
        addr[ni] = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds::lds_void*)(lb))) +
                   k0 * 512 + (((n >> 3) ^ (4 * (k0 & 3))) << 4) + (n & 7) * 2;
      }
      u32x2 r[8];  // r[4 ni + 2 ks + half]
      read_a(0);
      read_a(1);
      asm volatile(
          "ds_read_b64_tr_b16 %0, %8\n"
          "ds_read_b64_tr_b16 %1, %8 offset:2048\n"
          "ds_read_b64_tr_b16 %2, %8 offset:8192\n"
          "ds_read_b64_tr_b16 %3, %8 offset:10240\n"
          "ds_read_b64_tr_b16 %4, %9\n"
          "ds_read_b64_tr_b16 %5, %9 offset:2048\n"
          "ds_read_b64_tr_b16 %6, %9 offset:8192\n"
          "ds_read_b64_tr_b16 %7, %9 offset:10240\n"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]),
            "=&v"(r[6]), "=&v"(r[7])
          : "v"(addr[0]), "v"(addr[1])
          : "memory");
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
          const u32x2 lo = r[4 * ni + 2 * ks], hi = r[4 * ni + 2 * ks + 1];
          fb[ks][ni] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
    }
  };

  f32x16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const uint32_t nk = K / KB;
  const int grp = wave >> 2;
  // One K step (FILL: a refill exists, so the body has no branches).  Barrier
  // j of the workgroup closes group 0's phase j and group 1's phase j - 1: group
  // 0 reads stage k in [B(2k-1), B(2k)) and computes in [B(2k), B(2k+1)), group 1
  // one phase later.  Buffer (k-1) % NS is read by nobody after B(2k-1), so both
  // groups refill it in their compute phase of step k.  Every wave waits for its
  // share of stage k+1 at the end of its memory phase of step k, which precedes
  // B(2k+1), the barrier after which group 0 reads stage k+1.
  auto step = [&](uint32_t k, auto fill) {
    constexpr bool FILL = decltype(fill)::value;
    __builtin_amdgcn_sched_barrier(0);
    load_frags(k % NS);
    lds::wait_lgkm0();
    if constexpr (FILL) {
      // issued so far: stages up to k - 2 + NS; those past k + 1 stay in flight
      wait_vm<(NS - 3) * 2 * NLA>();
    } else if (k + 1 < nk) {
      const uint32_t last = min(nk - 1, max(k + NS - 2, static_cast<uint32_t>(NS - 1)));
      wait_stages<2 * NLA, NS - 2>(last - (k + 1));
    }
    bar();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (FILL) issue((k - 1) % NS, k - 1 + NS);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
          acc[mi][ni] = mfma32x32x16<DT>(fa[ks][mi], fb[ks][ni], acc[mi][ni]);
    __builtin_amdgcn_sched_barrier(0);
    bar();
  };

  // A previous work item of this workgroup (grid-stride callers) may still be
  // reading the arena in its epilogue.
  bar();
#pragma unroll
  for (uint32_t s = 0; s < NS; ++s)
    if (s < nk) issue(s, s);
  wait_stages<2 * NLA, NS - 1>(min(nk - 1, static_cast<uint32_t>(NS - 1)));
  bar();
  if (grp == 1) bar();
  uint32_t kt = 0;
  if (kt < nk) step(kt++, std::false_type{});
  for (; kt + NS - 1 < nk; ++kt) step(kt, std::true_type{});
  for (; kt < nk; ++kt) step(kt, std::false_type{});
  __builtin_amdgcn_sched_barrier(0);

  // Epilogue.  Accumulator register r of lane l in a 32x32 block holds row
  // 8*(r/4) + 4*(l/32) + r%4, column l%32: a lane has four consecutive rows of
  // one column, so direct stores are 2- or 4-byte writes (64-128 contiguous
  // bytes per row and instruction).  For a plain store that is as fast as any
  // rearrangement (measured): the tile's HBM writes bound it.  Each store keeps
  // its own bounds test, so stores leave one at a time between address updates:
  // at 4096^3 that is 4 us faster than issuing each 32x32 block's sixteen stores
  // back to back (measured on one box, same schedule otherwise).  Both groups
  // store after group 1's last compute phase: letting group 0 store during it was
  // 3 us slower.
  if (grp == 0) bar();
  if constexpr (EPI != kEpiSiluMul) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        const uint32_t col = n0 + wn * TWN + ni * 32 + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t row = m0 + wm * 128 + mi * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          if (row < M && col < N)
            store_out<EPI, DT_OUT>(C, up, static_cast<size_t>(row) * N + col, acc[mi][ni][r]);
        }
      }
    return;
  }
  // With the SiLU*Mul epilogue the UP operand makes scattered 2-byte reads as
  // well, so the tile goes through LDS: each wave parks 64 rows x 64 columns
  // of f32 at a time in a private 16 KB region of the idle stage arena and
  // reads them back as eight consecutive columns per lane.  UP and C then move
  // in 16-byte pieces (128 contiguous bytes per row and instruction), and UP's
  // loads are issued before the LDS round trip.
  // Region layout [64 r][64 c] f32, 4-float chunk q of row r at q ^ s(r) with
  // s(r) = (r & 1) | 8*((r >> 2) & 1): the scalar writes (rows r, r+4 across
  // the two lane halves) and the 16-byte reads (two rows per quarter-wave)
  // both cover all 64 banks.
  static_assert(TWN == 64 && 8 * 64 * 64 * 4 <= NS * (BM + BN) * KB * 2, "epilogue staging");
  constexpr int OSZ = (DT_OUT == kF32) ? 4 : 2;
  constexpr int UPV = 8 * OSZ / 16;  // 16-byte UP vectors per eight columns
  lds::wait_lgkm0();
  bar();  // every wave is done with the stage buffers
  float* wl = reinterpret_cast<float*>(arena) + wave * 64 * 64;
  auto sw = [](int r) { return (r & 1) | (((r >> 2) & 1) << 3); };
  const int rl = lane >> 3, cq = lane & 7;  // read-back: row rl + 8*it, columns 8*cq..+7
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t row0 = m0 + wm * 128 + 64 * h;
    const uint32_t col = n0 + wn * TWN + 8 * cq;
    // (N % 8 == 0 on this path: eight columns are either all inside or all past N)
    u32x4 upv[8][UPV];
#pragma unroll
    for (int it = 0; it < 8; ++it)
#pragma unroll
      for (int u = 0; u < UPV; ++u)
        upv[it][u] = (!edge || (row0 + rl + 8 * it < M && col < N))
                         ? ldg128(static_cast<const char*>(up) +
                                  ((static_cast<size_t>(row0 + rl + 8 * it) * N + col) * OSZ +
                                   16 * u))
                         : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int m2 = 0; m2 < 2; ++m2)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 32 * m2 + 8 * (r >> 2) + 4 * g + (r & 3);
          const int c = 32 * ni + l32;
          wl[row * 64 + (((c >> 2) ^ sw(row)) << 2) + (c & 3)] = acc[2 * h + m2][ni][r];
        }
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int row = rl + 8 * it;
      const f32x4 lo = *reinterpret_cast<const f32x4*>(wl + row * 64 + (((2 * cq) ^ sw(row)) << 2));
      const f32x4 hi =
          *reinterpret_cast<const f32x4*>(wl + row * 64 + (((2 * cq + 1) ^ sw(row)) << 2));
      float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      float u[8];
      if constexpr (DT_OUT == kF32) {
        // (__builtin_bit_cast straight from a vector element reads element 0 with
        // this compiler; the element goes through a scalar first)
#pragma unroll
        for (int e = 0; e < 8; ++e) u[e] = __uint_as_float(upv[it][e >> 2][e & 3]);
      } else {
        unpack16<DT_OUT>(upv[it][0], u);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = v[e] / (1.0f + expf(-v[e])) * u[e];
      if (edge && !(row0 + row < M && col < N)) continue;
      char* cp = static_cast<char*>(C) + (static_cast<size_t>(row0 + row) * N + col) * OSZ;
      if constexpr (DT_OUT == kF32) {
        stg128_nt(cp, __builtin_bit_cast(u32x4, f32x4{v[0], v[1], v[2], v[3]}));
        stg128_nt(cp + 16, __builtin_bit_cast(u32x4, f32x4{v[4], v[5], v[6], v[7]}));
      } else {
        stg128_nt(cp, pack16<DT_OUT>(v));
      }
    }
  }
}

// K multiple of KB (any M, N).  Batch index = blockIdx.y.
template <int DT, int DT_OUT, bool B_TRANS, int KB = gemm::DBK, int NS = gemm::NSTAGE,
          int WAVES = gemm::DWAVES, int EPI = 0, int MI = 4>
__global__ void __launch_bounds__(64 * WAVES, 1)
gemm_dma_256(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, void* __restrict__ C,
             uint32_t M, uint32_t N, uint32_t K, uint64_t sa, uint64_t sb, uint64_t sc,
             const void* __restrict__ up, uint32_t ldk) {
  uint32_t tm, tn;
  gemm::tile_coords(blockIdx.x, (M + gemm::BM - 1) / gemm::BM, (N + gemm::BN - 1) / gemm::BN, tm,
                    tn);
  constexpr int OSZ = (DT_OUT == kF32) ? 4 : 2;
  const size_t co = static_cast<size_t>(blockIdx.y) * sc * OSZ;
  gemm_dma_tile_256<DT, DT_OUT, B_TRANS, KB, NS, WAVES, EPI, MI>(
      A + blockIdx.y * sa, B + blockIdx.y * sb, static_cast<char*>(C) + co, M, N, K, tm, tn,
      up ? static_cast<const char*>(up) + co : nullptr, ldk);
}

// Split-K merge: C = epilogue(sum_s W[s]) for an S x M x N f32 workspace whose
// slice s holds A[:, s-th K range] . B[s-th K range, :].  Slices are added in
// ascending order; one rounding to C's dtype.
template <int DT_OUT, int EPI>
__global__ void __launch_bounds__(256)
gemm_splitk_reduce(const float* __restrict__ W, void* __restrict__ C, const void* __restrict__ up,
                   uint64_t mn, uint32_t S) {
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x; i < mn;
       i += static_cast<uint64_t>(gridDim.x) * 256u) {
    float v = 0.0f;
    for (uint32_t s = 0; s < S; ++s) v += W[s * mn + i];
    gemm::store_out<EPI, DT_OUT>(C, up, i, v);
  }
}

// Per-element GEMM on one 256x256 tile: each thread forms whole dot products
// with scalar loads, no LDS and no barriers, so it can stand in for any tile
// kernel whatever its workgroup size or LDS use.  Correctness fallback only (for
// operands the vector paths cannot take); f32 accumulation in k order.
template <int DT, int DT_OUT, bool B_TRANS, int EPI = 0>
__device__ __forceinline__ void gemm_dot_tile_256(const uint16_t* __restrict__ A,
                                                  const uint16_t* __restrict__ B,
                                                  void* __restrict__ C, uint32_t M, uint32_t N,
                                                  uint32_t K, uint32_t tm, uint32_t tn,
                                                  const void* __restrict__ up = nullptr) {
  for (uint32_t e = threadIdx.x; e < gemm::BM * gemm::BN; e += blockDim.x) {
    const uint32_t row = tm * gemm::BM + e / gemm::BN, col = tn * gemm::BN + e % gemm::BN;
    if (row >= M || col >= N) continue;
    float acc = 0.0f;
    for (uint32_t k = 0; k < K; ++k) {
      const float a = u16_to_f32<DT>(A[static_cast<size_t>(row) * K + k]);
      const float b = u16_to_f32<DT>(B_TRANS ? B[static_cast<size_t>(col) * K + k]
                                             : B[static_cast<size_t>(k) * N + col]);
      acc = __builtin_fmaf(a, b, acc);
    }
    gemm::store_out<EPI, DT_OUT>(C, up, static_cast<size_t>(row) * N + col, acc);
  }
}

// Fallback for 16-bit shapes the MFMA paths do not take (K % 8 != 0, row-major B
// with N % 8 != 0): 64x64 tile per 256-thread workgroup, each thread a 4x4 block,
// K staged 16 at a time through LDS, f32 FMA.
template <int DT, int DT_OUT, bool B_TRANS, int EPI = 0>
__device__ __forceinline__ void gemm_fma_tile_64(const void* __restrict__ A,
                                                 const void* __restrict__ B, void* __restrict__ C,
                                                 uint32_t M, uint32_t N, uint32_t K, uint32_t tile,
                                                 const void* __restrict__ up = nullptr) {
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
      if (row < M && col < N)
        gemm::store_out<EPI, DT_OUT>(C, up, static_cast<size_t>(row) * N + col, acc[i][j]);
    }
}

template <int DT, int DT_OUT, bool B_TRANS, int EPI = 0>
__global__ void __launch_bounds__(256)
gemm_fma_64(const void* __restrict__ A, const void* __restrict__ B, void* __restrict__ C,
            uint32_t M, uint32_t N, uint32_t K, uint64_t sa, uint64_t sb, uint64_t sc,
            const void* __restrict__ up) {
  constexpr int ISZ = (DT == kF32) ? 4 : 2;
  constexpr int OSZ = (DT_OUT == kF32) ? 4 : 2;
  const size_t co = static_cast<size_t>(blockIdx.y) * sc * OSZ;
  gemm_fma_tile_64<DT, DT_OUT, B_TRANS, EPI>(static_cast<const char*>(A) + blockIdx.y * sa * ISZ,
                                             static_cast<const char*>(B) + blockIdx.y * sb * ISZ,
                                             static_cast<char*>(C) + co, M, N, K, blockIdx.x,
                                             up ? static_cast<const char*>(up) + co : nullptr);
}

}  // namespace th

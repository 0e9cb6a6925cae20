// Device-side entry points for kernels emitted by the `hip` codegen target.
//
// An emitted tile kernel is a thin extern "C" __global__ wrapper around one of
// these.  Each loops over its work items grid-stride (item w is handled by
// workgroup w mod gridDim.x), so results never depend on the hardware grid the
// launcher picks from the kernel's launch descriptor; the descriptor only sizes
// the grid.  (One exception: the decode splits each sequence over as many
// workgroups as the grid allows, and the split changes the summation order.)  Per-tile pointer offsets follow the #[tile_kernel] prelude: logical
// tile t sees every view offset by t * rows * cols of that view
// (crates/tile_std_macros/src/lib.rs:217-266).
#pragma once

#include "../launch_desc.hpp"
#include "attention.hpp"
#include "attention_f32.hpp"
#include "common.hpp"
#include "gemm.hpp"
#include "gemm_asm.hpp"
#include "gemm_f32.hpp"
#include "norm.hpp"
#include "prefill_asm.hpp"
#include "softmax.hpp"

#ifndef TH_BUILD_STAMP
#define TH_BUILD_STAMP "unstamped"
#endif
// Every emitted code object carries the hash of the sources it was compiled
// from (passed by the build), so a test can check that the code object it loads
// was built from the tree it runs in.
extern "C" __device__ __attribute__((used)) const char __th_build_stamp[] = "th-src:" TH_BUILD_STAMP;

namespace th {
namespace entry {

// ---- row softmax over `rows` contiguous rows of `cols` (one wavefront per row;
//      rows of up to 256 16-byte vectors take the streaming loop of the library
//      kernel: each wave walks several rows with its next row's loads in flight) ----
// STREAM = false (pipelined_for(1), the explicit opt-out of pipelining) keeps one
// row per wave with no next row in flight.
template <int DT, int NV, bool STREAM = true>
__device__ __forceinline__ void softmax_rows(const void* x, void* y, uint32_t rows, uint32_t cols) {
  if constexpr (STREAM && NV > 0 && NV <= 4) {
    softmax_rows_stream_body<DT, NV>(x, y, rows, cols);
    return;
  }
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  const uint32_t wpg = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  for (uint32_t r = blockIdx.x * wpg + (threadIdx.x >> 6); r < rows; r += gridDim.x * wpg) {
    const size_t off = static_cast<size_t>(r) * cols * ESZ;
    const char* xr = static_cast<const char*>(x) + off;
    char* yr = static_cast<char*>(y) + off;
    if constexpr (NV > 0) softmax_row_wave<DT, NV>(xr, yr, cols, lane);
    else softmax_row_wave_any<DT>(xr, yr, cols, lane);
  }
}

// ---- rows of 1025-4096 16-byte vectors: one 256-thread workgroup per row, the
//      row in registers (workgroups stride over the rows) ----
template <int DT, int NV>
__device__ __forceinline__ void softmax_rows_wg(const void* x, void* y, uint32_t rows,
                                                uint32_t cols) {
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  for (uint32_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const size_t off = static_cast<size_t>(r) * cols * ESZ;
    softmax_row_wg<DT, NV>(static_cast<const char*>(x) + off, static_cast<char*>(y) + off, cols);
  }
}
template <int DT, int NV>
__device__ __forceinline__ void rms_norm_rows_wg(const void* x, void* y, uint32_t rows,
                                                 uint32_t cols, float eps) {
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  for (uint32_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const size_t off = static_cast<size_t>(r) * cols * ESZ;
    rms_norm_row_wg<DT, NV>(static_cast<const char*>(x) + off, static_cast<char*>(y) + off, cols,
                            eps);
  }
}

// ---- row RMSNorm over `rows` contiguous rows of `cols`: the library's streaming
//      loop when a row fits NV 16-byte vectors per lane (NV > 0), else one
//      wavefront per row in two passes ----
template <int DT, int NV = 0>
__device__ __forceinline__ void rms_norm_rows(const void* x, void* y, uint32_t rows, uint32_t cols,
                                              float eps) {
  if constexpr (NV > 0) {
    rms_norm_rows_stream_body<DT, NV>(x, y, rows, cols, eps);
    return;
  }
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  const uint32_t wpg = blockDim.x >> 6;
  for (uint32_t r = blockIdx.x * wpg + (threadIdx.x >> 6); r < rows; r += gridDim.x * wpg) {
    const size_t off = static_cast<size_t>(r) * cols * ESZ;
    rms_norm_row_wave_any<DT>(static_cast<const char*>(x) + off, static_cast<char*>(y) + off, cols,
                              eps, threadIdx.x & 63);
  }
}

// ---- batched GEMM: `batch` stacked problems, dense strides; EPI = gemm::kEpi* ----
// (kEpiSiluMul: C = silu(A.B) * UP, UP laid out like C)
template <int DT, int DTO, bool BT, int EPI = gemm::kEpiStore>
__device__ __forceinline__ void gemm(const uint16_t* A, const uint16_t* B, void* C, uint32_t M,
                                     uint32_t N, uint32_t K, uint32_t batch,
                                     const void* up = nullptr) {
  constexpr int OSZ = (DTO == kF32) ? 4 : 2;
  const uint32_t tiles_m = (M + gemm::BM - 1) / gemm::BM, tiles_n = (N + gemm::BN - 1) / gemm::BN;
  const uint32_t per = tiles_m * tiles_n;
  for (uint32_t w = blockIdx.x; w < per * batch; w += gridDim.x) {
    const uint32_t bi = w / per;
    uint32_t tm, tn;
    gemm::tile_coords(w % per, tiles_m, tiles_n, tm, tn);
    const size_t co = static_cast<size_t>(bi) * M * N * OSZ;
    gemm_tile_256<DT, DTO, BT, false, 2, 2, EPI>(
        A + static_cast<size_t>(bi) * M * K, B + static_cast<size_t>(bi) * K * N,
        static_cast<char*>(C) + co, M, N, K, tm, tn,
        up ? static_cast<const char*>(up) + co : nullptr);
  }
}

// Same contract on the LDS-DMA pipeline (8 waves: 512 threads per workgroup)
// for K a multiple of 32 (and N of 8).  Operands that are not 16-byte aligned
// (checked at run time; the emitter fixes only the view offsets) take the
// per-element kernel instead, which fits in the same workgroup.
// NS: LDS ring stages (4 or 5: the staged epilogue needs four stages of LDS).
template <int DT, int DTO, bool BT, int EPI = gemm::kEpiStore, int NS = gemm::NSTAGE>
__device__ __forceinline__ void gemm_dma(const uint16_t* A, const uint16_t* B, void* C, uint32_t M,
                                         uint32_t N, uint32_t K, uint32_t batch,
                                         const void* up = nullptr) {
  constexpr int OSZ = (DTO == kF32) ? 4 : 2;
  const uint32_t tiles_m = (M + gemm::BM - 1) / gemm::BM, tiles_n = (N + gemm::BN - 1) / gemm::BN;
  const uint32_t per = tiles_m * tiles_n;
  const size_t sa = static_cast<size_t>(M) * K * 2, sb = static_cast<size_t>(K) * N * 2;
  const size_t sc = static_cast<size_t>(M) * N * OSZ;
  const uintptr_t bits = reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B) |
                         reinterpret_cast<uintptr_t>(C) | reinterpret_cast<uintptr_t>(up) | sa |
                         sb | sc;
  const bool vec = (bits & 15) == 0;
  for (uint32_t w = blockIdx.x; w < per * batch; w += gridDim.x) {
    const uint32_t bi = w / per;
    uint32_t tm, tn;
    gemm::tile_coords(w % per, tiles_m, tiles_n, tm, tn);
    const uint16_t* a = A + static_cast<size_t>(bi) * M * K;
    const uint16_t* b = B + static_cast<size_t>(bi) * K * N;
    char* c = static_cast<char*>(C) + bi * sc;
    const void* u = up ? static_cast<const char*>(up) + bi * sc : nullptr;
    if (vec)
      gemm_dma_tile_256<DT, DTO, BT, gemm::DBK, NS, gemm::DWAVES, EPI>(a, b, c, M, N, K, tm, tn,
                                                                      u);
    else
      gemm_dot_tile_256<DT, DTO, BT, EPI>(a, b, c, M, N, K, tm, tn, u);
  }
}

// Whole 256 x 256 tiles with K a multiple of 128 (gasm::fits, checked by the emitter):
// the library's generated-assembly tile program, 256 threads per workgroup; SILU: the
// SiLU*Mul program (16-bit C, UP laid out like C).  Operands that are not 16-byte
// aligned (checked at run time) take the per-element kernel instead, which fits in the
// same workgroup.
template <int DT, int DTO, bool BT = false, bool SILU = false>
__device__ __forceinline__ void gemm_asm(const uint16_t* A, const uint16_t* B, void* C, uint32_t M,
                                         uint32_t N, uint32_t K, uint32_t batch,
                                         const void* up = nullptr) {
  constexpr int OSZ = (DTO == kF32) ? 4 : 2;
  const uint32_t tiles_m = M / 256, tiles_n = N / 256;
  const uint32_t per = tiles_m * tiles_n;
  const size_t sa = static_cast<size_t>(M) * K * 2, sb = static_cast<size_t>(K) * N * 2;
  const size_t sc = static_cast<size_t>(M) * N * OSZ;
  const uintptr_t bits = reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B) |
                         reinterpret_cast<uintptr_t>(C) | reinterpret_cast<uintptr_t>(up) | sa |
                         sb | sc;
  const bool vec = (bits & 15) == 0;
  if (vec && gridDim.x >= per * batch) {
    // One tile per workgroup (the launcher's grid) on a path that returns: the asm
    // statement clobbers most registers, and values live across it (the loop's state
    // below) are spilled to scratch and reloaded before every tile.
    const uint32_t w = blockIdx.x;
    if (w >= per * batch) return;
    const uint32_t bi = w / per;
    uint32_t tm, tn;
    gemm::tile_coords(w % per, tiles_m, tiles_n, tm, tn);
    gemm_asm_tile<DT, DTO, BT, SILU>(A + static_cast<size_t>(bi) * M * K,
                                     B + static_cast<size_t>(bi) * K * N,
                                     static_cast<char*>(C) + bi * sc, M, N, K, tm, tn,
                                     SILU ? static_cast<const char*>(up) + bi * sc : nullptr);
    return;
  }
  for (uint32_t w = blockIdx.x; w < per * batch; w += gridDim.x) {
    const uint32_t bi = w / per;
    uint32_t tm, tn;
    gemm::tile_coords(w % per, tiles_m, tiles_n, tm, tn);
    const uint16_t* a = A + static_cast<size_t>(bi) * M * K;
    const uint16_t* b = B + static_cast<size_t>(bi) * K * N;
    char* c = static_cast<char*>(C) + bi * sc;
    const void* u = SILU ? static_cast<const char*>(up) + bi * sc : nullptr;
    if (vec) {
      __syncthreads();  // the previous tile's last fragment reads (or UP reads) are done
      gemm_asm_tile<DT, DTO, BT, SILU>(a, b, c, M, N, K, tm, tn, u);
    } else {
      gemm_dot_tile_256<DT, DTO, BT, SILU ? gemm::kEpiSiluMul : gemm::kEpiStore>(a, b, c, M, N, K,
                                                                               tm, tn, u);
    }
  }
}

// ---- f32 operands: the fp32 MFMA kernel, 128 x 128 tiles (tiles of one
//      batch entry in XCD-grouped order) ----
template <int DTO, bool BT, bool VEC, int EPI = gemm::kEpiStore>
__device__ __forceinline__ void gemm_f32(const float* A, const float* B, void* C, uint32_t M,
                                         uint32_t N, uint32_t K, uint32_t batch,
                                         const void* up = nullptr) {
  constexpr int OSZ = (DTO == kF32) ? 4 : 2;
  const uint32_t tiles_m = (M + gf32::BM - 1) / gf32::BM, tiles_n = (N + gf32::BN - 1) / gf32::BN;
  const uint32_t per = tiles_m * tiles_n;
  // the 16-byte path also needs 16-byte aligned bases (the views' offsets are)
  const bool vec = VEC && ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 15) == 0;
  for (uint32_t w = blockIdx.x; w < per * batch; w += gridDim.x) {
    const uint32_t bi = w / per;
    uint32_t tm, tn;
    gemm::tile_coords<gf32::GROUP_M>(w % per, tiles_m, tiles_n, tm, tn);
    const size_t co = static_cast<size_t>(bi) * M * N * OSZ;
    const float* a = A + static_cast<size_t>(bi) * M * K;
    const float* b = B + static_cast<size_t>(bi) * K * N;
    const void* u = up ? static_cast<const char*>(up) + co : nullptr;
    if (vec) gemm_f32_tile_128<DTO, BT, true, EPI>(a, b, static_cast<char*>(C) + co, M, N, K, tm, tn, u);
    else gemm_f32_tile_128<DTO, BT, false, EPI>(a, b, static_cast<char*>(C) + co, M, N, K, tm, tn, u);
    __syncthreads();  // the LDS buffers are refilled by the next tile
  }
}

template <int DT, int DTO, bool BT, int EPI = gemm::kEpiStore>
__device__ __forceinline__ void gemm_fma(const void* A, const void* B, void* C, uint32_t M,
                                         uint32_t N, uint32_t K, uint32_t batch,
                                         const void* up = nullptr) {
  constexpr int ISZ = (DT == kF32) ? 4 : 2;
  constexpr int OSZ = (DTO == kF32) ? 4 : 2;
  const uint32_t per = ((M + 63) / 64) * ((N + 63) / 64);
  for (uint32_t w = blockIdx.x; w < per * batch; w += gridDim.x) {
    const uint32_t bi = w / per;
    const size_t co = static_cast<size_t>(bi) * M * N * OSZ;
    gemm_fma_tile_64<DT, DTO, BT, EPI>(
        static_cast<const char*>(A) + static_cast<size_t>(bi) * M * K * ISZ,
        static_cast<const char*>(B) + static_cast<size_t>(bi) * K * N * ISZ,
        static_cast<char*>(C) + co, M, N, K, w % per,
        up ? static_cast<const char*>(up) + co : nullptr);
  }
}

// ---- single-head non-causal attention on S x D tiles (__tile_attention_f32) ----
// f32 tiles with head_dim 64 or 128 and 16-byte aligned views run the fp32 MFMA
// flash kernel (one item per 128 queries); others one workgroup per query.
template <int DT, int NT>
__device__ __forceinline__ void attention_tiles(const void* q, const void* k, const void* v,
                                                void* o, uint32_t s, uint32_t d, uint32_t tiles) {
  const float scale = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(d)));
  if constexpr (DT == kF32) {
    const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                            reinterpret_cast<uintptr_t>(v);
    if ((d == 64 || d == 128) && (align & 15) == 0 && s > 0) {
      const uint32_t nqb = (s + af32::BQ - 1) / af32::BQ;
      auto Q = static_cast<const float*>(q);
      auto K = static_cast<const float*>(k);
      auto V = static_cast<const float*>(v);
      auto O = static_cast<float*>(o);
      const uint32_t total = tiles * nqb;
      for (uint32_t w = blockIdx.x; w < total; w += gridDim.x) {
        // one item per workgroup: XCD-grouped order (as the library kernel)
        const uint32_t it = gridDim.x == total ? af32::xcd_item(w, total) : w;
        if (d == 64) attn_f32_tile<64>(Q, K, V, O, s, scale * kLog2e, it / nqb, it % nqb);
        else attn_f32_tile<128>(Q, K, V, O, s, scale * kLog2e, it / nqb, it % nqb);
      }
      return;
    }
  }
  for (uint32_t w = blockIdx.x; w < tiles * s; w += gridDim.x)
    attn_general_item<DT, NT>(q, k, v, o, s, 0, s, s, d, 1, 1, 0, scale, w);
}

// ---- causal GQA prefill; runtime params in the Metal target's order ----
// HM: Q and O head-major, [B][NH][S][D] (the gpu emitter's __tile_attention_gqa_*,
// mlir_to_gpu.rs:1627-1712), instead of [B][S][NH][D].
template <int DT, bool HM = false>
__device__ __forceinline__ void prefill(const void* q, const void* k, const void* v, void* o,
                                        uint32_t batch, uint32_t seq_len, uint32_t start_pos,
                                        uint32_t max_seq, uint32_t head_dim, uint32_t nh,
                                        uint32_t nkv) {
  if (nkv == 0 || nh % nkv != 0 || start_pos + seq_len > max_seq || head_dim == 0 ||
      seq_len == 0)
    return;
  const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(head_dim));
  // the library's kernel (512 threads, the whole LDS as its K/V ring); the general
  // path below borrows the start of the same arena
  u32x4* arena = lds::dma_lds_arena<pfa::NS * 2 * pfa::BKV * pfa::D * 2>();
  if constexpr (DT != kF32) {
    const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                            reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(o);
    if ((head_dim == pfa::D || head_dim == 64) && (align & 15) == 0) {
      const uint32_t nqb = (seq_len + pfa::BQ - 1) / pfa::BQ;
      auto qq = static_cast<const uint16_t*>(q);
      auto kk = static_cast<const uint16_t*>(k);
      auto vv = static_cast<const uint16_t*>(v);
      auto oo = static_cast<uint16_t*>(o);
      if (gridDim.x >= batch * nh * nqb) {
        // One item per workgroup (the launcher's grid), each head dim on a path of its
        // own that returns: the asm statement clobbers v16-v255 and s48-s95, and values
        // live across it (the loop's state below) or shared by the two paths' operand
        // math are spilled to scratch around every item (2-3% at config 4).
        if (blockIdx.x >= batch * nh * nqb) return;
        if (head_dim == pfa::D) {
          // the same value as `scale` at head_dim 128 (sqrt and divide correctly rounded)
          const float s128 = 1.0f / __builtin_sqrtf(static_cast<float>(pfa::D));
          uint32_t bh, qb;
          prefill_work(blockIdx.x, batch, nh, nkv, nqb, bh, qb);
          pfa::prefill_tile<DT>(qq, kk, vv, oo, seq_len, start_pos, max_seq, nh, nkv,
                                s128 * kLog2e, bh, qb, HM);
          return;
        }
        uint32_t bh, qb;
        prefill_work(blockIdx.x, batch, nh, nkv, nqb, bh, qb);
        pfa::prefill_tile<DT, false, 64>(qq, kk, vv, oo, seq_len, start_pos, max_seq, nh, nkv,
                                         scale * kLog2e, bh, qb, HM);
        return;
      }
      for (uint32_t w = blockIdx.x; w < batch * nh * nqb; w += gridDim.x) {
        uint32_t bh, qb;
        prefill_work(w, batch, nh, nkv, nqb, bh, qb);
        if (head_dim == 64)
          pfa::prefill_tile<DT, false, 64>(qq, kk, vv, oo, seq_len, start_pos, max_seq, nh, nkv,
                                           scale * kLog2e, bh, qb, HM);
        else
          pfa::prefill_tile<DT>(qq, kk, vv, oo, seq_len, start_pos, max_seq, nh, nkv,
                                scale * kLog2e, bh, qb, HM);
        __syncthreads();  // every wave is done with the ring before the next item's DMA
      }
      return;
    }
  }
  static_assert(gen_attn::smem_floats<pfa::NT>() * 4 <= pfa::NS * 2 * pfa::BKV * pfa::D * 2,
                "general path's LDS inside the arena");
  if (head_dim <= 256) {
    for (uint32_t w = blockIdx.x; w < batch * seq_len * nh; w += gridDim.x)
      attn_general_item_smem<DT, pfa::NT>(q, k, v, o, seq_len, start_pos, max_seq,
                                          start_pos + seq_len, head_dim, nh, nkv, 1, scale, w,
                                          reinterpret_cast<float*>(arena), HM);
  }
}

// ---- GQA decode, one query token; runtime params in the Metal target's order ----
//
// KV split inside one launch: the (batch, kv_head) items are split into
// n_split = ceil(gridDim / items) chunk ranges (at most kDecodeMaxSplit, and
// only as many as the partials area holds); every split writes its partial
// (m, l, O) to `decode_partials`, counts itself in `decode_arrivals[item]`, and
// the workgroup that arrives last merges the item's partials into O and resets
// the count for the next launch.  The launcher sizes the grid to about two
// workgroups per CU, so one long sequence spreads over the whole chip while a
// large batch runs unsplit (one workgroup per item).
//
// The partials and counters are arrays of this code object in GPU memory: calls
// of one decode kernel that overlap on a device (other streams) race on them.
namespace dsplit {
constexpr uint32_t kMaxSplit = 64;                 // chunk ranges per item
constexpr uint32_t kMaxItems = 4096;               // counters: split items per launch
constexpr size_t kPartialFloats = size_t(2) << 20; // 8 MiB of partial records
}  // namespace dsplit
static __device__ __align__(256) float decode_partials[dsplit::kPartialFloats];
static __device__ uint32_t decode_arrivals[dsplit::kMaxItems];

// O rows of item bk = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s over its
// n_split records (as decode_tile writes them), for all G heads of the item.
template <int DT, int G, int HD = dec::D>
__device__ __forceinline__ void decode_merge(const float* __restrict__ ws, uint16_t* __restrict__ O,
                                             uint32_t bk, uint32_t nh, uint32_t nkv,
                                             uint32_t n_split) {
  constexpr int D = HD, NT = dec::NT, R = D + 2;
  constexpr int NP = G * D / 2;                  // output pairs (d, d+1)
  constexpr int NG = NP >= NT ? 1 : NT / NP;     // thread groups splitting the records
  constexpr int UNR = 8;
  __shared__ float s_w[G][dsplit::kMaxSplit];
  __shared__ float s_den[G];
  __shared__ float2 s_part[NG > 1 ? NG : 1][NG > 1 ? NP : 1];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const float* base = ws + static_cast<size_t>(bk) * G * n_split * R;
  for (int q = wave; q < G; q += NT / 64) {
    const float* rq = base + static_cast<size_t>(q) * n_split * R;
    const bool has = static_cast<uint32_t>(lane) < n_split;
    const float m = has ? rq[lane * R] : -INFINITY;
    const float l = has ? rq[lane * R + 1] : 0.0f;
    const float M = wave_max(m);
    const float w = (m == -INFINITY) ? 0.0f : exp2_fast(m - M);
    if (has) s_w[q][lane] = w;
    const float den = wave_sum(w * l);
    if (lane == 0) s_den[q] = den;
  }
  __syncthreads();
  const uint32_t b = bk / nkv, kvh = bk % nkv;
  for (int i = t % (NG > 1 ? NP : NT); i < NP; i += (NG > 1 ? NP : NT)) {
    const int q = i / (D / 2), d = 2 * (i % (D / 2));
    const int grp = NG > 1 ? t / NP : 0;
    const float* rd = base + static_cast<size_t>(q) * n_split * R + 2 + d;
    float2 acc = {0.0f, 0.0f};
    uint32_t s = grp;
    for (; s + (UNR - 1) * NG < n_split; s += UNR * NG) {
      float2 o[UNR];
#pragma unroll
      for (int u = 0; u < UNR; ++u) o[u] = *reinterpret_cast<const float2*>(rd + (s + u * NG) * R);
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const float w = s_w[q][s + u * NG];
        acc.x = __builtin_fmaf(w, o[u].x, acc.x);
        acc.y = __builtin_fmaf(w, o[u].y, acc.y);
      }
    }
    for (; s < n_split; s += NG) {
      const float2 o = *reinterpret_cast<const float2*>(rd + s * R);
      acc.x = __builtin_fmaf(s_w[q][s], o.x, acc.x);
      acc.y = __builtin_fmaf(s_w[q][s], o.y, acc.y);
    }
    if constexpr (NG > 1) {
      s_part[grp][i] = acc;
    } else {
      const float den = s_den[q];
      uint16_t* op = O + (static_cast<size_t>(b) * nh + kvh * G + q) * D + d;
      op[0] = f32_to_u16<DT>(den > 0.0f ? acc.x / den : 0.0f);
      op[1] = f32_to_u16<DT>(den > 0.0f ? acc.y / den : 0.0f);
    }
  }
  if constexpr (NG > 1) {
    __syncthreads();
    for (int i = t; i < NP; i += NT) {
      const int q = i / (D / 2), d = 2 * (i % (D / 2));
      float2 acc = s_part[0][i];
#pragma unroll
      for (int g = 1; g < NG; ++g) {
        acc.x += s_part[g][i].x;
        acc.y += s_part[g][i].y;
      }
      const float den = s_den[q];
      uint16_t* op = O + (static_cast<size_t>(b) * nh + kvh * G + q) * D + d;
      op[0] = f32_to_u16<DT>(den > 0.0f ? acc.x / den : 0.0f);
      op[1] = f32_to_u16<DT>(den > 0.0f ? acc.y / den : 0.0f);
    }
  }
  __syncthreads();  // s_w / s_den / s_part are reused by the next item
}

template <int DT, int G, int HD = dec::D>
__device__ __forceinline__ void decode_group(const uint16_t* q, const uint16_t* k,
                                             const uint16_t* v, uint16_t* o, uint32_t batch,
                                             uint32_t seq_len, uint32_t max_seq, uint32_t nh,
                                             uint32_t nkv, float scale_log2) {
  const uint32_t nchunks = (seq_len + dec::CHUNK - 1) / dec::CHUNK;
  const uint32_t items = batch * nkv;
  uint32_t n_split = (gridDim.x + items - 1) / items;
  n_split = min(n_split, min(nchunks, dsplit::kMaxSplit));
  const size_t per_split = static_cast<size_t>(items) * G * (HD + 2);
  n_split = min(static_cast<size_t>(n_split), dsplit::kPartialFloats / per_split);
  if (items > dsplit::kMaxItems || n_split < 2) n_split = 1;
  const uint32_t cps = (nchunks + n_split - 1) / n_split;
  n_split = (nchunks + cps - 1) / cps;   // no empty split
  __shared__ uint32_t s_last;
  for (uint32_t w = blockIdx.x; w < items * n_split; w += gridDim.x) {
    const uint32_t bk = w / n_split, split = w % n_split;
    const uint32_t c0 = split * cps, c1 = min(nchunks, c0 + cps);
    // unsplit: the workgroup covers the whole sequence and writes O itself
    // one LDS arena for every (G, HD) this kernel may run: the largest, not the sum
    decode_tile<DT, G, 4, 8, HD, 8, dec::D>(q, k, v, o, n_split > 1 ? decode_partials : nullptr,
                                            seq_len, max_seq, nh, nkv, n_split, scale_log2, bk,
                                            split, c0, c1);
    if (n_split == 1) continue;
    // decode_tile ends on a barrier: every wave's partial stores are issued.  The
    // release fence makes them visible device-wide before the arrival counts.
    if (threadIdx.x == 0) {
      __threadfence();
      s_last = atomicAdd(&decode_arrivals[bk], 1u) == n_split - 1;
    }
    __syncthreads();
    if (s_last) {
      __threadfence();   // acquire: the other splits' partials
      decode_merge<DT, G, HD>(decode_partials, o, bk, nh, nkv, n_split);
      if (threadIdx.x == 0) decode_arrivals[bk] = 0;   // ready for the next launch
    }
    __syncthreads();   // s_last is rewritten by the next item
  }
}

// The MFMA decode for head_dim HD (128 or 64); false: no instance for this group size.
template <int DT, int HD>
__device__ __forceinline__ bool decode_mfma(uint32_t g, const uint16_t* Q, const uint16_t* K,
                                            const uint16_t* V, uint16_t* O, uint32_t batch,
                                            uint32_t seq_len, uint32_t max_seq, uint32_t nh,
                                            uint32_t nkv, float sl2) {
  switch (g) {
    case 1: decode_group<DT, 1, HD>(Q, K, V, O, batch, seq_len, max_seq, nh, nkv, sl2); return true;
    case 2: decode_group<DT, 2, HD>(Q, K, V, O, batch, seq_len, max_seq, nh, nkv, sl2); return true;
    case 4: decode_group<DT, 4, HD>(Q, K, V, O, batch, seq_len, max_seq, nh, nkv, sl2); return true;
    case 8: decode_group<DT, 8, HD>(Q, K, V, O, batch, seq_len, max_seq, nh, nkv, sl2); return true;
    default: return false;
  }
}

template <int DT>
__device__ __forceinline__ void decode(const void* q, const void* k, const void* v, void* o,
                                       uint32_t batch, uint32_t seq_len, uint32_t max_seq,
                                       uint32_t head_dim, uint32_t nh, uint32_t nkv) {
  if (nkv == 0 || nh % nkv != 0 || seq_len > max_seq || head_dim == 0 || head_dim > 256) return;
  const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(head_dim));
  const uint32_t g = nh / nkv;
  if constexpr (DT != kF32) {
    if ((head_dim == dec::D || head_dim == 64) && seq_len > 0) {
      const float sl2 = scale * kLog2e;
      auto Q = static_cast<const uint16_t*>(q);
      auto K = static_cast<const uint16_t*>(k);
      auto V = static_cast<const uint16_t*>(v);
      auto O = static_cast<uint16_t*>(o);
      if (head_dim == 64 ? decode_mfma<DT, 64>(g, Q, K, V, O, batch, seq_len, max_seq, nh, nkv, sl2)
                         : decode_mfma<DT, dec::D>(g, Q, K, V, O, batch, seq_len, max_seq, nh, nkv,
                                                   sl2))
        return;
    }
  }
  for (uint32_t w = blockIdx.x; w < batch * nh; w += gridDim.x)
    attn_general_item<DT, dec::NT>(q, k, v, o, 1, 0, max_seq, seq_len, head_dim, nh, nkv, 0,
                                   scale, w);
}

// ---- row reductions of f32 rows (crates/rustc_codegen_tile/src/mlir_to_linalg.rs:
//      1496-1573 sum / max / absmax, :1576-1660 argmax): `tiles` x R rows of C
//      values -> one value per row, written at y[t * out_stride + r] (the stored
//      view of tile t starts t * out_stride elements in).  One wavefront per row;
//      lanes stride over 16-byte vectors when the row allows it. ----
enum RowReduce : int { kRowSum = 0, kRowMax = 1, kRowAbsMax = 2, kRowArgMax = 3 };

template <int OP>
__device__ __forceinline__ void row_reduce_step(float v, uint32_t c, float& acc, uint32_t& idx) {
  if constexpr (OP == kRowSum) acc += v;
  else if constexpr (OP == kRowMax) acc = maximumf(acc, v);        // reduce arith.maximumf
  else if constexpr (OP == kRowAbsMax) acc = maximumf(acc, fabsf(v));
  else if (v > acc) { acc = v; idx = c; }   // strict: the first index of the maximum
}

template <int OP>
__device__ __forceinline__ void reduce_rows(const float* __restrict__ x, float* __restrict__ y,
                                            uint32_t tiles, uint32_t R, uint32_t C,
                                            uint64_t out_stride) {
  const uint32_t wpg = blockDim.x >> 6;
  const uint32_t lane = threadIdx.x & 63;
  const uint64_t rows = static_cast<uint64_t>(tiles) * R;
  const bool vec = (C % 4 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0);
  for (uint64_t r = static_cast<uint64_t>(blockIdx.x) * wpg + (threadIdx.x >> 6); r < rows;
       r += static_cast<uint64_t>(gridDim.x) * wpg) {
    const float* xr = x + r * C;
    float acc = OP == kRowSum ? 0.0f : -INFINITY;
    uint32_t idx = 0;
    if (vec) {
      for (uint32_t c4 = lane; c4 < C / 4; c4 += 64) {
        const float4 v = reinterpret_cast<const float4*>(xr)[c4];
        row_reduce_step<OP>(v.x, 4 * c4, acc, idx);
        row_reduce_step<OP>(v.y, 4 * c4 + 1, acc, idx);
        row_reduce_step<OP>(v.z, 4 * c4 + 2, acc, idx);
        row_reduce_step<OP>(v.w, 4 * c4 + 3, acc, idx);
      }
    } else {
      for (uint32_t c = lane; c < C; c += 64) row_reduce_step<OP>(xr[c], c, acc, idx);
    }
    float* yr = y + (r / R) * out_stride + (r % R);
    if constexpr (OP == kRowArgMax) {
      for (int m = 1; m < 64; m <<= 1) {
        const float ov = __shfl_xor(acc, m);
        const uint32_t oi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(idx), m));
        if (ov > acc || (ov == acc && oi < idx)) {
          acc = ov;
          idx = oi;
        }
      }
      if (lane == 0) *reinterpret_cast<int32_t*>(yr) = static_cast<int32_t>(idx);
    } else {
      acc = OP == kRowSum ? wave_sum(acc) : wave_maximum(acc);
      if (lane == 0) *yr = acc;
    }
  }
}

// ---- transpose (mlir_to_linalg.rs:1458-1490): each tile's R x C f32 -> C x R,
//      32 x 32 blocks staged through LDS so that reads and writes are both
//      row-contiguous (256 threads) ----
__device__ __forceinline__ void transpose(const float* __restrict__ x, float* __restrict__ y,
                                          uint32_t tiles, uint32_t R, uint32_t C) {
  __shared__ float blk[32][33];
  const uint32_t br = (R + 31) / 32, bc = (C + 31) / 32;
  const uint64_t per = static_cast<uint64_t>(br) * bc;
  const uint32_t tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (uint64_t w = blockIdx.x; w < static_cast<uint64_t>(tiles) * per; w += gridDim.x) {
    const uint64_t t = w / per;
    const uint32_t b = static_cast<uint32_t>(w % per);
    const uint32_t r0 = (b / bc) * 32, c0 = (b % bc) * 32;
    const float* xt = x + t * R * C;
    float* yt = y + t * R * C;
    for (uint32_t i = ty; i < 32; i += 8) {
      const uint32_t r = r0 + i, c = c0 + tx;
      if (r < R && c < C) blk[i][tx] = xt[static_cast<uint64_t>(r) * C + c];
    }
    __syncthreads();
    for (uint32_t i = ty; i < 32; i += 8) {
      const uint32_t c = c0 + i, r = r0 + tx;
      if (r < R && c < C) yt[static_cast<uint64_t>(c) * R + r] = blk[tx][i];
    }
    __syncthreads();
  }
}

// ---- matvec (mlir_to_linalg.rs:1395-1440): y[R] = A[R x C] . x[C] per tile (A at
//      t*R*C, x at t*x_stride, y at t*y_stride), f32, one wavefront per row ----
__device__ __forceinline__ void matvec(const float* __restrict__ a, const float* __restrict__ x,
                                       float* __restrict__ y, uint32_t tiles, uint32_t R,
                                       uint32_t C, uint64_t x_stride, uint64_t y_stride) {
  const uint32_t wpg = blockDim.x >> 6;
  const uint32_t lane = threadIdx.x & 63;
  const uint64_t rows = static_cast<uint64_t>(tiles) * R;
  for (uint64_t r = static_cast<uint64_t>(blockIdx.x) * wpg + (threadIdx.x >> 6); r < rows;
       r += static_cast<uint64_t>(gridDim.x) * wpg) {
    const uint64_t t = r / R;
    const float* ar = a + r * C;
    const float* xt = x + t * x_stride;
    float acc = 0.0f;
    for (uint32_t c = lane; c < C; c += 64) acc = __builtin_fmaf(ar[c], xt[c], acc);
    acc = wave_sum(acc);
    if (lane == 0) y[t * y_stride + (r % R)] = acc;
  }
}

}  // namespace entry
}  // namespace th

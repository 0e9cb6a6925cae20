// Single-head, non-causal attention on f32 S x D tiles on the fp32 matrix cores
// (v_mfma_f32_32x32x2_f32): the __tile_attention_f32 op (crates/tile_std/src/
// tile.rs:221, :2401; linalg semantics crates/rustc_codegen_tile/src/
// mlir_to_linalg.rs:1781-1902: O = softmax(Q K^T * scale) V, scale = 1/sqrt(D)
// rounded from f64 to f32).
//
// Flash form: one 256-thread workgroup per (tile, 128-query block), 32 queries
// per wave; K and V stream through LDS in blocks of 32 positions (two buffers,
// the next block prefetched into registers while the current one computes), and
// the softmax runs online with f32 row max and sum.
//
// Per 32-position block a wave computes S^T = K . Q^T as one 32 x 32 MFMA block:
// the A operand is K (lane l: position l % 32), the B operand Q^T lives in
// registers for the whole pass (lane l: query l % 32), so accumulator r of lane l
// is the score of query l % 32 at position f(r, h) = 8 (r / 4) + 4 h + r % 4,
// h = l / 32.  The row max needs one exchange between the lane halves.  The
// probabilities then feed O += P . V without moving: step r of the 16 MFMA steps
// takes position f(r, h) from lane half h, for P (A operand, registers) and V
// (B operand, LDS row f(r, h)) alike.  O's accumulator rows are queries, so the
// per-query rescale factors and final sums go through a 32-float LDS slot per
// wave.  The head dimension is split between lane halves in the S^T product as
// d = 4 (ks / 2) + 2 h + ks % 2, so a lane's K values for steps 2m and 2m+1 are
// adjacent (one 8-byte LDS read) and its Q^T registers fill from 16-byte loads of
// its query row.  In O += P . V, 32-column block c of O holds head dims
// d = ND n + c (n = l32, ND = D / 32 blocks), so a lane reads its V values for all
// blocks as ND adjacent floats (one 16-byte read at D 128) and writes its O row
// piece as one 16-byte store.
//
// LDS rows: K [32][D + 2] (an 8-byte read of positions 0..31 covers the 64 banks
// once per lane half), V [32][D] (each 16-byte read takes 128 contiguous bytes per
// eight lanes).  Reading K and V one float per lane, paired by the compiler into
// two-address reads, cost one bank-conflict cycle per MFMA (27% of LDS-active
// cycles).
//
// Work order: the 128-query blocks of one problem run on one XCD, so its K and V
// are read from HBM about once and then served by that XCD's L2.
#pragma once

#include "common.hpp"

namespace th {
namespace af32 {
constexpr int BQ = 128;   // queries per workgroup
constexpr int BKV = 32;   // positions per K/V block
constexpr int NT = 256;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// 16-byte aligned: V tiles go in, and the per-wave factors come out, as 16-byte LDS
// accesses
template <int D>
struct alignas(16) Lds {
  float k[2][BKV * (D + 2)];
  float v[2][BKV * D];
  float stat[NT / 64][32];   // per-wave query factors (rescale, then 1 / sum)
};
template <int D>
__device__ __forceinline__ Lds<D>& smem() {
  __shared__ Lds<D> s;
  return s;
}
}  // namespace af32

// Queries qb*128 .. +127 of problem `tile` (Q, K, V, O: [tiles][S][D] f32).
template <int D>
__device__ __forceinline__ void attn_f32_tile(const float* __restrict__ Q,
                                              const float* __restrict__ K,
                                              const float* __restrict__ V, float* __restrict__ O,
                                              uint32_t S, float scale_log2, uint32_t tile,
                                              uint32_t qb) {
  using namespace af32;
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  constexpr int LK = D + 2, LV = D;
  constexpr int KP = BKV * D / 2 / NT;   // float2 pieces of K per thread
  constexpr int VP = BKV * D / 4 / NT;   // float4 pieces of V per thread
  constexpr int ND = D / 32;             // 32-wide column blocks of O
  Lds<D>& s = smem<D>();
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const size_t base = static_cast<size_t>(tile) * S * D;
  const float* Kt = K + base;
  const float* Vt = V + base;

  // Q^T operand: q = q0 + 32 wave + l32 (rows past S read row S-1, not stored)
  const uint32_t q = qb * BQ + 32 * wave + l32;
  const uint32_t qc = min(q, S - 1);
  float qf[D / 2];
  {
    const float* qr = Q + base + static_cast<size_t>(qc) * D;
#pragma unroll
    for (int j = 0; j < D / 4; ++j) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(qr + 4 * j);
      qf[2 * j] = x[2 * h];
      qf[2 * j + 1] = x[2 * h + 1];
    }
  }

  f32x2 rk[KP];
  f32x4 rv[VP];
  auto load = [&](uint32_t kv0) {
#pragma unroll
    for (int i = 0; i < KP; ++i) {
      const int e = t + NT * i;               // piece e: row e / (D/2), cols 2 (e % (D/2))
      const uint32_t row = kv0 + e / (D / 2);
      rk[i] = row < S ? *reinterpret_cast<const f32x2*>(Kt + static_cast<size_t>(row) * D + 2 * (e % (D / 2)))
                      : f32x2{0.0f, 0.0f};
    }
#pragma unroll
    for (int i = 0; i < VP; ++i) {
      const int e = t + NT * i;
      const uint32_t row = kv0 + e / (D / 4);
      rv[i] = row < S ? *reinterpret_cast<const f32x4*>(Vt + static_cast<size_t>(row) * D + 4 * (e % (D / 4)))
                      : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KP; ++i) {
      const int e = t + NT * i;
      *reinterpret_cast<f32x2*>(&s.k[buf][(e / (D / 2)) * LK + 2 * (e % (D / 2))]) = rk[i];
    }
#pragma unroll
    for (int i = 0; i < VP; ++i) {
      const int e = t + NT * i;
      *reinterpret_cast<f32x4*>(&s.v[buf][(e / (D / 4)) * LV + 4 * (e % (D / 4))]) = rv[i];
    }
  };

  f32x16 acc[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;   // of query l32 (l_run: this half's share)

  const uint32_t nb = (S + BKV - 1) / BKV;
  load(0);
  store(0);
  __syncthreads();
  for (uint32_t jb = 0; jb < nb; ++jb) {
    const int cur = jb & 1;
    if (jb + 1 < nb) load((jb + 1) * BKV);
    // ---- S^T = K . Q^T ----
    f32x16 st;
#pragma unroll
    for (int r = 0; r < 16; ++r) st[r] = 0.0f;
    const float* kr = s.k[cur] + l32 * LK + 2 * h;
#pragma unroll
    for (int m = 0; m < D / 4; ++m) {
      const f32x2 k2 = *reinterpret_cast<const f32x2*>(kr + 4 * m);
      st = __builtin_amdgcn_mfma_f32_32x32x2f32(k2[0], qf[2 * m], st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_32x32x2f32(k2[1], qf[2 * m + 1], st, 0, 0, 0);
    }
    // ---- online softmax of query l32 over positions f(r, h) ----
    const uint32_t kv0 = jb * BKV;
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const uint32_t pos = kv0 + 8 * (r >> 2) + 4 * h + (r & 3);
      st[r] = pos < S ? st[r] * scale_log2 : -INFINITY;
      mx = fmaxf(mx, st[r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);    // finite: every block has a position < S
    const float alpha = exp2_fast(m_run - m_new);
    float sum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      st[r] = exp2_fast(st[r] - m_new);
      sum += st[r];
    }
    l_run = l_run * alpha + sum;
    m_run = m_new;
    // ---- O = O * alpha + P . V (O rows are queries: alpha through LDS) ----
    if (h == 0) s.stat[wave][l32] = alpha;
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): the wave's own LDS write
    __builtin_amdgcn_wave_barrier();
    {
      const f32x4* sa = reinterpret_cast<const f32x4*>(&s.stat[wave][4 * h]);
      f32x4 a4[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) a4[g] = sa[2 * g];   // queries 8 g + 4 h .. +3
#pragma unroll
      for (int c = 0; c < ND; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] *= a4[r >> 2][r & 3];
    }
    const float* vr = s.v[cur] + (4 * h) * LV + ND * l32;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float* vrow = vr + (8 * (r >> 2) + (r & 3)) * LV;
      float vv[ND];
      if constexpr (ND == 4) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(vrow);
#pragma unroll
        for (int c = 0; c < 4; ++c) vv[c] = x[c];
      } else {
        const f32x2 x = *reinterpret_cast<const f32x2*>(vrow);
        vv[0] = x[0];
        vv[1] = x[1];
      }
#pragma unroll
      for (int c = 0; c < ND; ++c)
        acc[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(st[r], vv[c], acc[c], 0, 0, 0);
    }
    if (jb + 1 < nb) store(cur ^ 1);
    __syncthreads();   // also orders this block's stat reads before the next writes
  }

  // ---- O / l, rows of the accumulator are queries 8 (r / 4) + 4 h + r % 4 ----
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (h == 0) s.stat[wave][l32] = 1.0f / l_tot;
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  const uint32_t qw = qb * BQ + 32 * wave;
  const bool o16 = (reinterpret_cast<uintptr_t>(O) & 15) == 0;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int qi = 8 * (r >> 2) + 4 * h + (r & 3);
    const float inv = s.stat[wave][qi];
    if (qw + qi < S) {
      // columns ND l32 .. ND l32 + ND - 1 of the row
      float* orow = O + base + static_cast<size_t>(qw + qi) * D + ND * l32;
      f32x4 ov;
#pragma unroll
      for (int c = 0; c < 4; ++c) ov[c] = c < ND ? acc[c < ND ? c : 0][r] * inv : 0.0f;
      if (ND == 4 && o16) {
        *reinterpret_cast<f32x4*>(orow) = ov;
      } else {
#pragma unroll
        for (int c = 0; c < ND; ++c) orow[c] = ov[c];
      }
    }
  }
  __syncthreads();   // LDS is reused by the next work item
}

namespace af32 {
// Work item of hardware block `bid` out of `total`: the hardware deals workgroups
// to the 8 XCDs round-robin, so item ids are renumbered to give each XCD a
// contiguous run (consecutive query blocks of one problem share its L2).
__device__ __forceinline__ uint32_t xcd_item(uint32_t bid, uint32_t total) {
  return total % 8 == 0 ? (bid % 8) * (total / 8) + bid / 8 : bid;
}
}  // namespace af32

// Library kernel: grid = tiles * ceil(S / 128), S >= 1.
template <int D>
__global__ void __launch_bounds__(af32::NT)
attn_f32_mfma(const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
              float* __restrict__ O, uint32_t S, float scale_log2) {
  const uint32_t nqb = (S + af32::BQ - 1) / af32::BQ;
  const uint32_t w = af32::xcd_item(blockIdx.x, gridDim.x);
  attn_f32_tile<D>(Q, K, V, O, S, scale_log2, w / nqb, w % nqb);
}

}  // namespace th

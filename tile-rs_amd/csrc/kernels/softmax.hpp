// Row softmax: y[r][c] = exp(x[r][c] - max_r) / sum_c exp(x[r][c] - max_r).
//
// Semantics: `linalg.softmax dimension(1)` as emitted for __tile_softmax_f32
// (reference: crates/rustc_codegen_tile/src/mlir_to_linalg.rs:1305-1343);
// intrinsic ABI (dst, src, rows, cols) at crates/tile_std/src/tile.rs:190, :2297;
// the f16 variant at tile.rs:2163, :2912.  Math is f32 for every I/O dtype.
//
// HBM-bound.  Each row is owned by one wavefront: the row is read once with
// 128-bit coalesced loads straight into registers, the max and the sum are
// 64-lane DPP/shuffle reductions, and the row is written once.  Rows too long
// for registers use a three-pass workgroup kernel instead.
#pragma once

#include "common.hpp"

namespace th {

// Register path: one wavefront owns one row; NV 16-byte vectors per lane, so a
// row holds up to 64 * NV * kElems elements.  Requires cols % kElems == 0 and
// 16-byte aligned rows.  xr / yr point at the row.
template <int DT, int NV>
__device__ __forceinline__ void softmax_row_wave(const void* __restrict__ xr_,
                                                 void* __restrict__ yr_, uint32_t cols, int lane) {
  constexpr int E = Vec16<DT>::kElems;
  const uint32_t nvec = cols / E;  // 16-byte vectors in this row
  const char* xr = static_cast<const char*>(xr_);
  char* yr = static_cast<char*>(yr_);

  float v[NV][E];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const uint32_t vi = static_cast<uint32_t>(i) * 64u + lane;
    if (vi < nvec) {
      unpack16<DT>(ldg128_nt(xr + static_cast<size_t>(vi) * 16), v[i]);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) v[i][e] = -INFINITY;
    }
  }
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < E; ++e) m = fmaxf(m, v[i][e]);
  m = wave_max(m);
  // exp(x - m) = exp2(x*log2e - m*log2e), one fused multiply-add per element.
  const float mb = m * kLog2e;
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float p = exp2_fast(__builtin_fmaf(v[i][e], kLog2e, -mb));
      v[i][e] = p;
      s += p;
    }
  s = wave_sum(s);
  const float inv = 1.0f / s;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const uint32_t vi = static_cast<uint32_t>(i) * 64u + lane;
    if (vi < nvec) {
#pragma unroll
      for (int e = 0; e < E; ++e) v[i][e] *= inv;
      stg128_nt(yr + static_cast<size_t>(vi) * 16, pack16<DT>(v[i]));
    }
  }
}

// Rows per workgroup = blockDim.x / 64.
template <int DT, int NV>
__global__ void __launch_bounds__(256)
softmax_rows_reg(const void* __restrict__ x, void* __restrict__ y, uint32_t rows, uint32_t cols) {
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  const uint32_t row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const size_t off = static_cast<size_t>(row) * cols * ESZ;
  softmax_row_wave<DT, NV>(static_cast<const char*>(x) + off, static_cast<char*>(y) + off, cols,
                           threadIdx.x & 63);
}

// Streaming form of the register path: a fixed grid of waves walks the rows
// (row stride = total waves), and the loads of a wave's next row are issued
// before the reductions of its current row, so every wave keeps one row of
// loads in flight.  Called by every thread of the workgroup (any grid size).
template <int DT, int NV>
__device__ __forceinline__ void softmax_rows_stream_body(const void* __restrict__ x,
                                                         void* __restrict__ y, uint32_t rows,
                                                         uint32_t cols) {
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  constexpr int E = Vec16<DT>::kElems;
  const int lane = threadIdx.x & 63;
  const uint32_t nvec = cols / E;
  const uint32_t stride = gridDim.x * (blockDim.x >> 6);
  uint32_t row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const size_t rbytes = static_cast<size_t>(cols) * ESZ;
  u32x4 cur[NV], nxt[NV];
  auto load = [&](uint32_t r, u32x4 (&v)[NV]) {
    const char* xr = static_cast<const char*>(x) + static_cast<size_t>(r) * rbytes;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t vi = static_cast<uint32_t>(i) * 64u + lane;
      // cached loads: 6-7% faster than nontemporal ones for this row stream (measured)
      if (vi < nvec) v[i] = ldg128(xr + static_cast<size_t>(vi) * 16);
    }
  };
  if (row < rows) load(row, cur);
  for (; row < rows; row += stride) {
    if (row + stride < rows) load(row + stride, nxt);
    float v[NV][E];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t vi = static_cast<uint32_t>(i) * 64u + lane;
      if (vi < nvec) {
        unpack16<DT>(cur[i], v[i]);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) v[i][e] = -INFINITY;
      }
#pragma unroll
      for (int e = 0; e < E; ++e) m = fmaxf(m, v[i][e]);
    }
    m = wave_max(m);
    const float mb = m * kLog2e;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float p = exp2_fast(__builtin_fmaf(v[i][e], kLog2e, -mb));
        v[i][e] = p;
        s += p;
      }
    s = wave_sum(s);
    const float inv = 1.0f / s;
    char* yr = static_cast<char*>(y) + static_cast<size_t>(row) * rbytes;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t vi = static_cast<uint32_t>(i) * 64u + lane;
      if (vi < nvec) {
#pragma unroll
        for (int e = 0; e < E; ++e) v[i][e] *= inv;
        stg128_nt(yr + static_cast<size_t>(vi) * 16, pack16<DT>(v[i]));
      }
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) cur[i] = nxt[i];
  }
}

template <int DT, int NV>
__global__ void __launch_bounds__(256)
softmax_rows_stream(const void* __restrict__ x, void* __restrict__ y, uint32_t rows,
                    uint32_t cols) {
  softmax_rows_stream_body<DT, NV>(x, y, rows, cols);
}

// Any cols, one wavefront per row, three passes over the row (no LDS).
template <int DT>
__device__ __forceinline__ float ld_elem(const void* p, size_t i);
template <int DT>
__device__ __forceinline__ void st_elem(void* p, size_t i, float v);

template <int DT>
__device__ __forceinline__ void softmax_row_wave_any(const void* __restrict__ xr,
                                                     void* __restrict__ yr, uint32_t cols,
                                                     int lane) {
  float m = -INFINITY;
  for (uint32_t c = lane; c < cols; c += 64) m = fmaxf(m, ld_elem<DT>(xr, c));
  m = wave_max(m);
  const float mb = m * kLog2e;
  float s = 0.0f;
  for (uint32_t c = lane; c < cols; c += 64)
    s += exp2_fast(__builtin_fmaf(ld_elem<DT>(xr, c), kLog2e, -mb));
  s = wave_sum(s);
  const float inv = 1.0f / s;
  for (uint32_t c = lane; c < cols; c += 64)
    st_elem<DT>(yr, c, exp2_fast(__builtin_fmaf(ld_elem<DT>(xr, c), kLog2e, -mb)) * inv);
}

// Generic path for any cols (ragged, unaligned or longer than the register path
// holds): one 256-thread workgroup per row, three passes over the row.
template <int DT>
__device__ __forceinline__ float ld_elem(const void* p, size_t i) {
  if constexpr (DT == kF32) return static_cast<const float*>(p)[i];
  else return u16_to_f32<DT>(static_cast<const uint16_t*>(p)[i]);
}
template <int DT>
__device__ __forceinline__ void st_elem(void* p, size_t i, float v) {
  if constexpr (DT == kF32) static_cast<float*>(p)[i] = v;
  else static_cast<uint16_t*>(p)[i] = f32_to_u16<DT>(v);
}

template <int DT>
__global__ void __launch_bounds__(256)
softmax_rows_generic(const void* __restrict__ x, void* __restrict__ y, uint32_t rows,
                     uint32_t cols) {
  __shared__ float red[4];
  const uint32_t row = blockIdx.x;
  if (row >= rows) return;
  const size_t base = static_cast<size_t>(row) * cols;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;

  float m = -INFINITY;
  for (uint32_t c = threadIdx.x; c < cols; c += 256) m = fmaxf(m, ld_elem<DT>(x, base + c));
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();

  const float mb = m * kLog2e;
  float s = 0.0f;
  for (uint32_t c = threadIdx.x; c < cols; c += 256)
    s += exp2_fast(__builtin_fmaf(ld_elem<DT>(x, base + c), kLog2e, -mb));
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  s = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.0f / s;

  for (uint32_t c = threadIdx.x; c < cols; c += 256)
    st_elem<DT>(y, base + c, exp2_fast(__builtin_fmaf(ld_elem<DT>(x, base + c), kLog2e, -mb)) * inv);
}

}  // namespace th

// Row RMSNorm: y[r][c] = x[r][c] * rsqrt(sum_c x[r][c]^2 / cols + eps).
//
// Semantics: `__tile_rms_norm_f32(dst, src, eps, rows, cols)` (reference:
// crates/tile_std/src/tile.rs:2063) as lowered by the linalg bridge
// (crates/rustc_codegen_tile/src/mlir_to_linalg.rs:1666-1763): square, sum
// over dimension 1, divide by cols, add eps, rsqrt, multiply.  Math is f32 for
// every I/O dtype (16-bit inputs are widened exactly, outputs rounded RNE).
//
// HBM-bound, same structure as the streaming softmax: a fixed grid of waves
// walks the rows, each row held in registers (128-bit nontemporal loads), the
// sum of squares a 64-lane reduction, one pass over HBM.  Longer rows use one
// workgroup per row or a chunked two-kernel pass (below).
#pragma once

#include "common.hpp"
#include "softmax.hpp"

namespace th {

// Called by every thread of the workgroup (any grid size).
template <int DT, int NV>
__device__ __forceinline__ void rms_norm_rows_stream_body(const void* __restrict__ x,
                                                          void* __restrict__ y, uint32_t rows,
                                                          uint32_t cols, float eps) {
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  constexpr int E = Vec16<DT>::kElems;
  const int lane = threadIdx.x & 63;
  const uint32_t nvec = cols / E;
  const uint32_t stride = gridDim.x * (blockDim.x >> 6);
  uint32_t row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const size_t rbytes = static_cast<size_t>(cols) * ESZ;
  const float inv_cols = 1.0f / static_cast<float>(cols);
  u32x4 cur[NV], nxt[NV];
  auto load = [&](uint32_t r, u32x4 (&v)[NV]) {
    const char* xr = static_cast<const char*>(x) + static_cast<size_t>(r) * rbytes;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t vi = static_cast<uint32_t>(i) * 64u + lane;
      v[i] = (vi < nvec) ? ldg128_nt(xr + static_cast<size_t>(vi) * 16) : u32x4{0, 0, 0, 0};
    }
  };
  if (row < rows) load(row, cur);
  for (; row < rows; row += stride) {
    if (row + stride < rows) load(row + stride, nxt);
    // Rows stay packed in registers (16 vectors per lane at most): the sum of
    // squares and the scaling each unpack on the fly.
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float v[E];
      unpack16<DT>(cur[i], v);
#pragma unroll
      for (int e = 0; e < E; ++e) ss = __builtin_fmaf(v[e], v[e], ss);
    }
    ss = wave_sum(ss);
    // mean = sum / cols; rsqrt(mean + eps)
    const float rs = 1.0f / __builtin_sqrtf(ss * inv_cols + eps);
    char* yr = static_cast<char*>(y) + static_cast<size_t>(row) * rbytes;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t vi = static_cast<uint32_t>(i) * 64u + lane;
      if (vi < nvec) {
        float v[E];
        unpack16<DT>(cur[i], v);
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] *= rs;
        stg128_nt(yr + static_cast<size_t>(vi) * 16, pack16<DT>(v));
      }
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) cur[i] = nxt[i];
  }
}

template <int DT, int NV>
__global__ void __launch_bounds__(256)
rms_norm_rows_stream(const void* __restrict__ x, void* __restrict__ y, uint32_t rows,
                     uint32_t cols, float eps) {
  rms_norm_rows_stream_body<DT, NV>(x, y, rows, cols, eps);
}

// Any cols / alignment: one wavefront per row, two passes over the row.
template <int DT>
__device__ __forceinline__ void rms_norm_row_wave_any(const void* __restrict__ xr,
                                                      void* __restrict__ yr, uint32_t cols,
                                                      float eps, int lane) {
  float ss = 0.0f;
  for (uint32_t c = lane; c < cols; c += 64) {
    const float v = ld_elem<DT>(xr, c);
    ss = __builtin_fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  const float rs = 1.0f / __builtin_sqrtf(ss * (1.0f / static_cast<float>(cols)) + eps);
  for (uint32_t c = lane; c < cols; c += 64) st_elem<DT>(yr, c, ld_elem<DT>(xr, c) * rs);
}

// Long rows.  With at least one row per CU and up to 4096 16-byte vectors per
// row: one 256-thread workgroup per row, the row in registers, a block-wide sum
// of squares (one read, one write).  Otherwise each row is cut into chunks
// spread over about four workgroups per CU: rms_norm_part_stats writes every
// chunk's sum of squares, rms_norm_part_apply adds its row's sums and scales
// the chunk (two reads, one write).
__device__ __forceinline__ float block_sum256(float v) {
  __shared__ float red[4];
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// Body: the calling workgroup normalizes the row at xr into yr (may be called
// again for another row).
template <int DT, int NV>
__device__ __forceinline__ void rms_norm_row_wg(const char* __restrict__ xr, char* __restrict__ yr,
                                                uint32_t cols, float eps) {
  constexpr int E = Vec16<DT>::kElems;
  const uint32_t nvec = cols / E;
  const int t = threadIdx.x;
  __syncthreads();  // a previous row's readers of the reduction slots are done
  float v[NV][E];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const uint32_t vi = static_cast<uint32_t>(i) * 256u + t;
    if (vi < nvec) {
      unpack16<DT>(ldg128_nt(xr + static_cast<size_t>(vi) * 16), v[i]);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) v[i][e] = 0.0f;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) ss = __builtin_fmaf(v[i][e], v[i][e], ss);
  }
  ss = block_sum256(ss);
  const float rs = 1.0f / __builtin_sqrtf(ss * (1.0f / static_cast<float>(cols)) + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const uint32_t vi = static_cast<uint32_t>(i) * 256u + t;
    if (vi < nvec) {
#pragma unroll
      for (int e = 0; e < E; ++e) v[i][e] *= rs;
      stg128_nt(yr + static_cast<size_t>(vi) * 16, pack16<DT>(v[i]));
    }
  }
}

template <int DT, int NV>
__global__ void __launch_bounds__(256)
rms_norm_rows_wg(const void* __restrict__ x, void* __restrict__ y, uint32_t rows, uint32_t cols,
                 float eps) {
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  const uint32_t row = blockIdx.x;
  if (row >= rows) return;
  const size_t off = static_cast<size_t>(row) * cols * ESZ;
  rms_norm_row_wg<DT, NV>(static_cast<const char*>(x) + off, static_cast<char*>(y) + off, cols,
                          eps);
}

template <int DT>
__global__ void __launch_bounds__(256)
rms_norm_part_stats(const void* __restrict__ x, float* __restrict__ st, uint32_t cols,
                    uint32_t parts, uint32_t chunk) {
  constexpr int E = Vec16<DT>::kElems;
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  const uint32_t row = blockIdx.x / parts, p = blockIdx.x % parts;
  const uint32_t c0 = p * chunk, c1 = min(cols, c0 + chunk);
  const size_t base = static_cast<size_t>(row) * cols;
  float ss = 0.0f;
  chunk_visit<ESZ, true>(
      static_cast<const char*>(x) + base * ESZ, c0, c1,
      [&](u32x4 raw, uint32_t) {
        float f[E];
        unpack16<DT>(raw, f);
#pragma unroll
        for (int e = 0; e < E; ++e) ss = __builtin_fmaf(f[e], f[e], ss);
      },
      [&](uint32_t c) {
        const float f = ld_elem<DT>(x, base + c);
        ss = __builtin_fmaf(f, f, ss);
      });
  ss = block_sum256(ss);
  if (threadIdx.x == 0) st[blockIdx.x] = ss;
}

// VEC: x and y have the same 16-byte phase (see softmax_part_apply).
template <int DT, bool VEC>
__global__ void __launch_bounds__(256)
rms_norm_part_apply(const void* x, void* y, const float* __restrict__ st, uint32_t cols,
                    uint32_t parts, uint32_t chunk, float eps) {
  constexpr int E = Vec16<DT>::kElems;
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  const uint32_t row = blockIdx.x / parts, p = blockIdx.x % parts;
  const uint32_t c0 = p * chunk, c1 = min(cols, c0 + chunk);
  const size_t base = static_cast<size_t>(row) * cols;
  float ss = 0.0f;
  for (uint32_t q = threadIdx.x; q < parts; q += 256) ss += st[static_cast<size_t>(row) * parts + q];
  ss = block_sum256(ss);
  const float rs = 1.0f / __builtin_sqrtf(ss * (1.0f / static_cast<float>(cols)) + eps);
  auto one = [&](uint32_t c) { st_elem<DT>(y, base + c, ld_elem<DT>(x, base + c) * rs); };
  if constexpr (VEC) {
    char* yr = static_cast<char*>(y) + base * ESZ;
    chunk_visit<ESZ, false>(
        static_cast<const char*>(x) + base * ESZ, c0, c1,
        [&](u32x4 raw, uint32_t c) {
          float f[E];
          unpack16<DT>(raw, f);
#pragma unroll
          for (int e = 0; e < E; ++e) f[e] *= rs;
          stg128_nt(yr + static_cast<size_t>(c) * ESZ, pack16<DT>(f));
        },
        one);
  } else {
    for (uint32_t c = c0 + threadIdx.x; c < c1; c += 256) one(c);
  }
}

}  // namespace th

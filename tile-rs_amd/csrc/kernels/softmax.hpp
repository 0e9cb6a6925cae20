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
// for one wavefront's registers use one workgroup per row (the row still in
// registers) or, for longer rows or few rows, a two-pass kernel pair over row
// chunks spread across the chip.
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

// Workgroup form of the register path (used by emitted kernels): one 256-thread
// workgroup per row, NV 16-byte vectors per thread (rows up to 4096 vectors:
// 16384 f32 or 32768 16-bit values), block-wide max and sum; one read and one
// write of the row.  The calling workgroup normalizes the row at xr into yr
// (every thread calls it; it may be called again for another row).
template <int DT, int NV>
__device__ __forceinline__ void softmax_row_wg(const char* __restrict__ xr, char* __restrict__ yr,
                                               uint32_t cols) {
  constexpr int E = Vec16<DT>::kElems;
  __shared__ float red[4];
  const uint32_t nvec = cols / E;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  __syncthreads();  // a previous row's readers of red[] are done
  float v[NV][E];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const uint32_t vi = static_cast<uint32_t>(i) * 256u + t;
    if (vi < nvec) {
      unpack16<DT>(ldg128_nt(xr + static_cast<size_t>(vi) * 16), v[i]);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) v[i][e] = -INFINITY;
    }
  }
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < E; ++e) m = fmaxf(m, v[i][e]);
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  const float mb = m * kLog2e;
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < E; ++e) {
      v[i][e] = exp2_fast(__builtin_fmaf(v[i][e], kLog2e, -mb));
      s += v[i][e];
    }
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  const float inv = 1.0f / ((red[0] + red[1]) + (red[2] + red[3]));
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const uint32_t vi = static_cast<uint32_t>(i) * 256u + t;
    if (vi < nvec) {
#pragma unroll
      for (int e = 0; e < E; ++e) v[i][e] *= inv;
      stg128_nt(yr + static_cast<size_t>(vi) * 16, pack16<DT>(v[i]));
    }
  }
}

// Streaming workgroup form: a fixed grid of NT-thread workgroups walks the rows
// (NV 16-byte vectors per thread, rows up to NT * NV vectors), and each
// workgroup's loads of its next row are issued before it reduces the current
// one, so no row's load latency is exposed.
template <int DT, int NT, int NV>
__global__ void __launch_bounds__(NT)
softmax_rows_wg_stream(const void* __restrict__ x, void* __restrict__ y, uint32_t rows,
                       uint32_t cols) {
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  constexpr int E = Vec16<DT>::kElems;
  constexpr int NW = NT / 64;
  __shared__ float red[NW];
  const uint32_t nvec = cols / E;
  const size_t rbytes = static_cast<size_t>(cols) * ESZ;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  u32x4 cur[NV], nxt[NV];
  auto load = [&](uint32_t r, u32x4 (&v)[NV]) {
    const char* xr = static_cast<const char*>(x) + static_cast<size_t>(r) * rbytes;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t vi = static_cast<uint32_t>(i) * NT + t;
      if (vi < nvec) v[i] = ldg128_nt(xr + static_cast<size_t>(vi) * 16);
    }
  };
  auto block_max = [&](float v) {
    v = wave_max(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) r = fmaxf(r, red[w]);
    __syncthreads();
    return r;
  };
  auto block_sum = [&](float v) {
    v = wave_sum(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) r += red[w];
    __syncthreads();
    return r;
  };
  uint32_t row = blockIdx.x;
  if (row < rows) load(row, cur);
  for (; row < rows; row += gridDim.x) {
    if (row + gridDim.x < rows) load(row + gridDim.x, nxt);
    float v[NV][E];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t vi = static_cast<uint32_t>(i) * NT + t;
      if (vi < nvec) {
        unpack16<DT>(cur[i], v[i]);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) v[i][e] = -INFINITY;
      }
#pragma unroll
      for (int e = 0; e < E; ++e) m = fmaxf(m, v[i][e]);
    }
    const float mb = block_max(m) * kLog2e;
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        v[i][e] = exp2_fast(__builtin_fmaf(v[i][e], kLog2e, -mb));
        sum += v[i][e];
      }
    const float inv = 1.0f / block_sum(sum);
    char* yr = static_cast<char*>(y) + static_cast<size_t>(row) * rbytes;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t vi = static_cast<uint32_t>(i) * NT + t;
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

// Scalar element access for ragged or unaligned rows.
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

// ---- long rows: each row split over `parts` workgroups --------------------------
// Rows too long for one wavefront's registers are cut into chunks of `chunk`
// elements so that every CU takes part whatever the row count:
//   softmax_part_stats: workgroup (row, p) reads chunk p once and writes its
//     statistics (m_p, s_p), m_p = max x (in log2 units), s_p = sum 2^(x - m_p);
//   softmax_part_apply: workgroup (row, p) merges its row's statistics,
//     M = max m_p, S = sum s_p 2^(m_p - M), and writes 2^(x - M) / S over chunk p.
// Two reads and one write of the row.  A row of -inf only gives NaN, as the
// single-pass kernels do.  Chunks are read with 16-byte loads between scalar
// head and tail columns, so ragged and unaligned rows keep most of the rate.

// Visit columns [c0, c1) of a row (element 0 at `row`), thread-strided over a
// 256-thread workgroup: scalar columns up to the first 16-byte boundary, then
// 16-byte vectors (four in flight per thread), then the scalar tail.  vec(raw,
// c) receives the vector starting at column c, one(c) a single column.
template <int ESZ, bool NT, class FV, class F1>
__device__ __forceinline__ void chunk_visit(const char* row, uint32_t c0, uint32_t c1, FV&& vec,
                                            F1&& one) {
  constexpr uint32_t E = 16 / ESZ;
  const char* s0 = row + static_cast<size_t>(c0) * ESZ;
  const uint32_t head =
      min(c1 - c0, static_cast<uint32_t>(((16u - (reinterpret_cast<uintptr_t>(s0) & 15u)) & 15u) / ESZ));
  const uint32_t cv = c0 + head;
  const uint32_t nv = (c1 - cv) / E;
  const char* sv = s0 + static_cast<size_t>(head) * ESZ;
  auto ld = [&](uint32_t v) { return NT ? ldg128_nt(sv + static_cast<size_t>(v) * 16)
                                        : ldg128(sv + static_cast<size_t>(v) * 16); };
  for (uint32_t c = c0 + threadIdx.x; c < cv; c += 256) one(c);
  constexpr int U = 4;
  uint32_t v = threadIdx.x;
  for (; v + 256 * (U - 1) < nv; v += 256 * U) {
    u32x4 raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) raw[u] = ld(v + 256 * u);
#pragma unroll
    for (int u = 0; u < U; ++u) vec(raw[u], cv + (v + 256 * u) * E);
  }
  for (; v < nv; v += 256) vec(ld(v), cv + v * E);
  for (uint32_t c = cv + nv * E + threadIdx.x; c < c1; c += 256) one(c);
}

// (m, s) pairs in log2 units: merge b into a.
__device__ __forceinline__ void stat_merge(float& m, float& s, float mb, float sb) {
  const float mx = fmaxf(m, mb);
  if (mx == -INFINITY) return;  // both empty
  s = s * exp2_fast(m - mx) + sb * exp2_fast(mb - mx);
  m = mx;
}

// Block-wide merge of every thread's (m, s); the result is valid in every thread.
__device__ __forceinline__ void block_stat_merge(float& m, float& s) {
  __shared__ float red_m[4], red_s[4];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1)
    stat_merge(m, s, __shfl_xor(m, off, 64), __shfl_xor(s, off, 64));
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red_m[wave] = m;
    red_s[wave] = s;
  }
  __syncthreads();
  m = red_m[0];
  s = red_s[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) stat_merge(m, s, red_m[w], red_s[w]);
}

template <int DT>
__global__ void __launch_bounds__(256)
softmax_part_stats(const void* __restrict__ x, float2* __restrict__ st, uint32_t cols,
                   uint32_t parts, uint32_t chunk) {
  constexpr int E = Vec16<DT>::kElems;
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  const uint32_t row = blockIdx.x / parts, p = blockIdx.x % parts;
  const uint32_t c0 = p * chunk, c1 = min(cols, c0 + chunk);
  const size_t base = static_cast<size_t>(row) * cols;
  float m = -INFINITY, s = 0.0f;
  // fold n values (already scaled to log2 units) into (m, s)
  auto fold = [&](const float* v, int n) {
    float vm = v[0];
    for (int i = 1; i < n; ++i) vm = fmaxf(vm, v[i]);
    if (vm == -INFINITY) return;
    if (vm > m) {
      s *= exp2_fast(m - vm);
      m = vm;
    }
    for (int i = 0; i < n; ++i) s += exp2_fast(v[i] - m);
  };
  chunk_visit<ESZ, true>(
      static_cast<const char*>(x) + base * ESZ, c0, c1,
      [&](u32x4 raw, uint32_t) {
        float f[E];
        unpack16<DT>(raw, f);
#pragma unroll
        for (int e = 0; e < E; ++e) f[e] *= kLog2e;
        fold(f, E);
      },
      [&](uint32_t c) {
        const float f = ld_elem<DT>(x, base + c) * kLog2e;
        fold(&f, 1);
      });
  block_stat_merge(m, s);
  if (threadIdx.x == 0) st[blockIdx.x] = make_float2(m, s);
}

// VEC: x and y have the same 16-byte phase, so the vector middle of each chunk
// is aligned for both; otherwise every column is scalar.
template <int DT, bool VEC>
__global__ void __launch_bounds__(256)
softmax_part_apply(const void* x, void* y, const float2* __restrict__ st, uint32_t cols,
                   uint32_t parts, uint32_t chunk) {
  constexpr int E = Vec16<DT>::kElems;
  constexpr int ESZ = (DT == kF32) ? 4 : 2;
  const uint32_t row = blockIdx.x / parts, p = blockIdx.x % parts;
  const uint32_t c0 = p * chunk, c1 = min(cols, c0 + chunk);
  const size_t base = static_cast<size_t>(row) * cols;
  float m = -INFINITY, s = 0.0f;
  for (uint32_t q = threadIdx.x; q < parts; q += 256) {
    const float2 v = st[static_cast<size_t>(row) * parts + q];
    stat_merge(m, s, v.x, v.y);
  }
  block_stat_merge(m, s);
  if (m == -INFINITY) s = NAN;  // a row of -inf: 0/0 as in the single-pass kernels
  const float inv = 1.0f / s;
  auto one = [&](uint32_t c) {
    st_elem<DT>(y, base + c, exp2_fast(__builtin_fmaf(ld_elem<DT>(x, base + c), kLog2e, -m)) * inv);
  };
  if constexpr (VEC) {
    char* yr = static_cast<char*>(y) + base * ESZ;
    chunk_visit<ESZ, false>(
        static_cast<const char*>(x) + base * ESZ, c0, c1,
        [&](u32x4 raw, uint32_t c) {
          float f[E];
          unpack16<DT>(raw, f);
#pragma unroll
          for (int e = 0; e < E; ++e) f[e] = exp2_fast(__builtin_fmaf(f[e], kLog2e, -m)) * inv;
          stg128_nt(yr + static_cast<size_t>(c) * ESZ, pack16<DT>(f));
        },
        one);
  } else {
    for (uint32_t c = c0 + threadIdx.x; c < c1; c += 256) one(c);
  }
}

}  // namespace th

// Device-side helpers shared by every tile-op kernel (gfx950 / CDNA4 only).
//
// The tile ops carry f16 and bf16 in the same u16 carrier
// (reference: crates/tile_std/src/lib.rs:182); the dtype is a runtime tag here.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace th {

// Element-type tags; numerically equal to TH_DTYPE_* in include/tilers_hip.h.
enum Dtype : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

// ---- 16-bit float conversions ------------------------------------------------
// Widening is exact; narrowing rounds to nearest even, matching `arith.extf` /
// `arith.truncf` in the reference's linalg bridge (mlir_to_linalg.rs:1249-1303).

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
    return static_cast<uint16_t>((u >> 16) | 0x0040u);
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return static_cast<float>(v);
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  _Float16 v = static_cast<_Float16>(f);  // v_cvt_f16_f32: round to nearest even
  return __builtin_bit_cast(uint16_t, v);
}

template <int DT>
__device__ __forceinline__ float u16_to_f32(uint16_t h) {
  if constexpr (DT == kBF16) return bf16_to_f32(h);
  else return f16_to_f32(h);
}

template <int DT>
__device__ __forceinline__ uint16_t f32_to_u16(float f) {
  if constexpr (DT == kBF16) return f32_to_bf16(f);
  else return f32_to_f16(f);
}

// Two f32 -> packed pair of 16-bit values (lo in bits 0..15).
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_u16<DT>(lo)) |
         (static_cast<uint32_t>(f32_to_u16<DT>(hi)) << 16);
}

// Elements in one 16-byte vector, and 16-byte vector <-> f32 conversions
// (exact widening, RNE narrowing).
template <int DT>
struct Vec16 {
  static constexpr int kElems = (DT == kF32) ? 4 : 8;  // elements per 16 B
};

template <int DT>
__device__ __forceinline__ void unpack16(u32x4 v, float (&f)[Vec16<DT>::kElems]) {
  if constexpr (DT == kF32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = u16_to_f32<DT>(static_cast<uint16_t>(v[i] & 0xffffu));
      f[2 * i + 1] = u16_to_f32<DT>(static_cast<uint16_t>(v[i] >> 16));
    }
  }
}

template <int DT>
__device__ __forceinline__ u32x4 pack16(const float (&f)[Vec16<DT>::kElems]) {
  u32x4 v;
  if constexpr (DT == kF32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __float_as_uint(f[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = pack2<DT>(f[2 * i], f[2 * i + 1]);
  }
  return v;
}

// ---- wavefront (64-lane) reductions ---------------------------------------------
// Lanes within a 16-lane row use DPP; the two cross-row steps use ds_swizzle-free
// lane shuffles.

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<0xb1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f32<0x4e>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f32<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_f32<0x140>(v));  // row_mirror
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

// IEEE 754-2019 maximum / minimum, the semantics of MLIR's arith.maximumf /
// arith.minimumf (and of linalg.max / linalg.min on floats): NaN when either
// operand is NaN, and -0 < +0.  gfx950 has them as v_maximum3_f32 / v_minimum3_f32.
// (fmaxf / fminf are maxNum / minNum: they drop a NaN operand.)
__device__ __forceinline__ float maximumf(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}
__device__ __forceinline__ float minimumf(float a, float b) {
  return __builtin_elementwise_minimum(a, b);
}

// wave_max with maximumf: a NaN in any lane reaches every lane
__device__ __forceinline__ float wave_maximum(float v) {
  v = maximumf(v, dpp_f32<0xb1>(v));
  v = maximumf(v, dpp_f32<0x4e>(v));
  v = maximumf(v, dpp_f32<0x141>(v));
  v = maximumf(v, dpp_f32<0x140>(v));
  v = maximumf(v, __shfl_xor(v, 16));
  v = maximumf(v, __shfl_xor(v, 32));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0xb1>(v);
  v += dpp_f32<0x4e>(v);
  v += dpp_f32<0x141>(v);
  v += dpp_f32<0x140>(v);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// exp(x) for x <= 0 via the hardware base-2 exponential.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- MFMA wrappers (gfx950) ---------------------------------------------------

template <int DT>
__device__ __forceinline__ f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == kBF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

template <int DT>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == kBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// Dword built from the low (SEL_HI=false) or high 16-bit halves of two dwords:
// result = lo_src.half | (hi_src.half << 16).
template <bool SEL_HI>
__device__ __forceinline__ uint32_t pack_halves(uint32_t lo_src, uint32_t hi_src) {
  return __builtin_amdgcn_perm(hi_src, lo_src, SEL_HI ? 0x07060302u : 0x05040100u);
}

// ---- global memory helpers -----------------------------------------------------

__device__ __forceinline__ u32x4 ldg128(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ u32x4 ldg128_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void stg128_nt(void* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// ---- LDS DMA pipeline helpers (gfx950) ------------------------------------------
namespace lds {
// LDS ring of a DMA-pipeline kernel (BYTES of gfx950's 160 KB per CU).
template <int BYTES>
__device__ __forceinline__ u32x4* dma_lds_arena() {
  static_assert(BYTES % 16 == 0 && BYTES <= 160 * 1024, "LDS arena");
  __shared__ u32x4 arena[BYTES / 16];
  return arena;
}
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

// Workgroup barrier without a memory fence: LDS DMA completion is handled by
// explicit vmcnt waits, and a fence would drain every outstanding load.
__device__ __forceinline__ void bar() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt bits [3:0] and [15:14]).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// s_waitcnt lgkmcnt(0)
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// global_load_lds_dwordx4: lane i copies 16 bytes from its own `src` to
// lds_dst + 16*i (lds_dst is the wave-uniform base).
__device__ __forceinline__ void dma16(const void* src, void* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)(lds_dst), 16, 0, 0);
}
// ds_read_b64_tr_b16: within each 16-lane group the lanes address a 4 x 16
// block of 16-bit values (4 rows, lane s pointing at row s/4, elements
// 4(s%4)..+3); lane i receives column i, rows 0..3.
__device__ __forceinline__ u32x2 read_tr16(const void* lds_addr) {
  const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(const_cast<void*>(lds_addr)));
  return __builtin_bit_cast(u32x2, v);
}
}  // namespace lds

}  // namespace th

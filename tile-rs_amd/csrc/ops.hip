// Tile-op entry points of the C ABI (include/tilers_hip.h, section 2); the GEMM ones
// (th_matmul, th_matmul_silu_mul) are in ops_gemm.hip.
//
// Each entry point checks shapes and pointers on the host, picks the
// hand-written gfx950 kernel for the shape, and enqueues it on the caller's
// stream.  There is no CPU fallback: a shape no kernel takes is an error.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>

#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <mutex>
#include <string>
#include <type_traits>

#include "kernels/attention.hpp"
#include "kernels/attention_f32.hpp"
#include "kernels/prefill_asm.hpp"
#include "kernels/common.hpp"
#include "kernels/norm.hpp"
#include "kernels/softmax.hpp"
#include "ops_common.hpp"
#include "runtime.hpp"

using th::fail;
using namespace th::ops;

namespace {

// ---- softmax ----------------------------------------------------------------

// Rows longer than the register paths hold (or ragged / unaligned rows): each row
// is cut into chunks (a multiple of 8 elements, at least 2048) so that about
// four workgroups per CU run; one pass writes every chunk's (max, sum) to a
// per-stream statistics buffer, the second merges a row's statistics and
// writes the chunk.  Measured on MI355X against one workgroup per row with
// scalar loads: 64 x 131072 f32 411 -> 21 us, 1 x 2^20 f32 2708 -> 9 us.
template <int DT>
int softmax_long(const void* x, void* y, uint32_t rows, uint32_t cols, hipStream_t s) {
  const uint64_t target = 4ull * current_cu_count();
  uint64_t parts = std::max<uint64_t>(1, (target + rows - 1) / rows);
  parts = std::min<uint64_t>(parts, (cols + 2047) / 2048);
  uint64_t chunk = (cols + parts - 1) / parts;
  chunk = (chunk + 7) / 8 * 8;
  parts = (cols + chunk - 1) / chunk;
  const uint64_t blocks = static_cast<uint64_t>(rows) * parts;
  if (blocks > 0x7fffffffu) return fail(TH_KERNEL_ERROR, "softmax: grid too large");
  void* stv = nullptr;
  TH_TRY(th::stream_scratch(s, blocks * sizeof(float2), &stv));
  auto* st = static_cast<float2*>(stv);
  const dim3 grid(static_cast<uint32_t>(blocks)), block(256);
  const uint32_t P = static_cast<uint32_t>(parts), Cn = static_cast<uint32_t>(chunk);
  hipLaunchKernelGGL((th::softmax_part_stats<DT>), grid, block, 0, s, x, st, cols, P, Cn);
  if (same_phase16(x, y))
    hipLaunchKernelGGL((th::softmax_part_apply<DT, true>), grid, block, 0, s, x, y, st, cols, P,
                       Cn);
  else
    hipLaunchKernelGGL((th::softmax_part_apply<DT, false>), grid, block, 0, s, x, y, st, cols, P,
                       Cn);
  return launch_status("softmax launch");
}

template <int DT>
int softmax_launch(const void* x, void* y, uint32_t rows, uint32_t cols, hipStream_t s) {
  constexpr int E = th::Vec16<DT>::kElems;
  const bool vec_ok = (cols % E == 0) && aligned16(x) && aligned16(y);
  const uint32_t nvec = cols / E;
  if (vec_ok && nvec <= 64u * 4u) {
    // Streaming form: 4 workgroups (16 waves) per CU walk the rows; measured
    // on MI355X this sustains the copy-kernel bandwidth, while one short-lived
    // wave per row does not.
    const uint32_t need = (rows + 3) / 4;
    // two workgroups per CU: each wave streams several rows, next row in flight
    const dim3 grid(std::min<uint32_t>(need, 2u * current_cu_count())), block(256);
    if (nvec <= 64)
      hipLaunchKernelGGL((th::softmax_rows_stream<DT, 1>), grid, block, 0, s, x, y, rows, cols);
    else if (nvec <= 128)
      hipLaunchKernelGGL((th::softmax_rows_stream<DT, 2>), grid, block, 0, s, x, y, rows, cols);
    else
      hipLaunchKernelGGL((th::softmax_rows_stream<DT, 4>), grid, block, 0, s, x, y, rows, cols);
    return launch_status("softmax launch");
  }
  if (vec_ok && nvec > 64u * 8u && nvec <= 512u * 8u && rows >= current_cu_count()) {
    // enough rows to fill the chip: a fixed grid of workgroups walks the rows,
    // each row in registers and the next row's loads in flight.  Measured on
    // MI355X against one wave per row: 1024-vector rows 36.8 -> 30.5 us
    // (4096 x 8192 bf16); 512-vector rows stay faster on one wave per row.
    const uint32_t cus = current_cu_count();
    if (nvec <= 256u * 4u) {
      const dim3 grid(std::min<uint32_t>(rows, 2u * cus)), block(256);
      hipLaunchKernelGGL((th::softmax_rows_wg_stream<DT, 256, 4>), grid, block, 0, s, x, y, rows,
                         cols);
    } else if (nvec <= 256u * 8u) {
      const dim3 grid(std::min<uint32_t>(rows, 2u * cus)), block(256);
      hipLaunchKernelGGL((th::softmax_rows_wg_stream<DT, 256, 8>), grid, block, 0, s, x, y, rows,
                         cols);
    } else {
      const dim3 grid(std::min<uint32_t>(rows, 2u * cus)), block(512);
      hipLaunchKernelGGL((th::softmax_rows_wg_stream<DT, 512, 8>), grid, block, 0, s, x, y, rows,
                         cols);
    }
    return launch_status("softmax launch");
  }
  if (vec_ok && nvec <= 64u * 16u) {
    const uint32_t rows_per_wg = 4;
    const dim3 grid((rows + rows_per_wg - 1) / rows_per_wg), block(256);
    if (nvec <= 512)
      hipLaunchKernelGGL((th::softmax_rows_reg<DT, 8>), grid, block, 0, s, x, y, rows, cols);
    else
      hipLaunchKernelGGL((th::softmax_rows_reg<DT, 16>), grid, block, 0, s, x, y, rows, cols);
  } else {
    return softmax_long<DT>(x, y, rows, cols, s);
  }
  return launch_status("softmax launch");
}

// Streaming row kernels: as many 256-thread workgroups as fit on every CU at
// once (at most 4), so the grid is one resident wave of work with no tail.
template <class K>
uint32_t resident_grid(K kernel, int* cache, uint32_t rows) {
  if (*cache == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, 256, 0) != hipSuccess || n <= 0)
      n = 1;
    *cache = std::min(n, 4);
  }
  return std::max(1u, std::min<uint32_t>((rows + 3) / 4,
                                         static_cast<uint32_t>(*cache) * current_cu_count()));
}

template <int DT, int NV>
void rms_norm_stream_go(const void* x, void* y, uint32_t rows, uint32_t cols, float eps,
                        hipStream_t s) {
  static int per_cu = 0;
  auto k = th::rms_norm_rows_stream<DT, NV>;
  hipLaunchKernelGGL(k, dim3(resident_grid(k, &per_cu, rows)), dim3(256), 0, s, x, y, rows, cols,
                     eps);
}

template <int DT>
int rms_norm_launch(const void* x, void* y, uint32_t rows, uint32_t cols, float eps,
                    hipStream_t s) {
  constexpr int E = th::Vec16<DT>::kElems;
  const bool vec_ok = (cols % E == 0) && aligned16(x) && aligned16(y);
  const uint32_t nvec = cols / E;
  if (vec_ok && nvec <= 64) rms_norm_stream_go<DT, 1>(x, y, rows, cols, eps, s);
  else if (vec_ok && nvec <= 128) rms_norm_stream_go<DT, 2>(x, y, rows, cols, eps, s);
  else if (vec_ok && nvec <= 256) rms_norm_stream_go<DT, 4>(x, y, rows, cols, eps, s);
  else if (vec_ok && nvec <= 512) rms_norm_stream_go<DT, 8>(x, y, rows, cols, eps, s);
  else if (vec_ok && nvec <= 1024) rms_norm_stream_go<DT, 16>(x, y, rows, cols, eps, s);
  else if (vec_ok && nvec <= 256u * 16u && rows >= current_cu_count()) {
    // enough rows to fill the chip: one workgroup per row, the row in registers
    if (nvec <= 256u * 8u)
      hipLaunchKernelGGL((th::rms_norm_rows_wg<DT, 8>), dim3(rows), dim3(256), 0, s, x, y, rows,
                         cols, eps);
    else
      hipLaunchKernelGGL((th::rms_norm_rows_wg<DT, 16>), dim3(rows), dim3(256), 0, s, x, y, rows,
                         cols, eps);
  } else {
    // long, ragged or unaligned rows: chunk sums of squares, then scale (as softmax_long)
    const uint64_t target = 4ull * current_cu_count();
    uint64_t parts = std::max<uint64_t>(1, (target + rows - 1) / rows);
    parts = std::min<uint64_t>(parts, (cols + 2047) / 2048);
    uint64_t chunk = (cols + parts - 1) / parts;
    chunk = (chunk + 7) / 8 * 8;
    parts = (cols + chunk - 1) / chunk;
    const uint64_t blocks = static_cast<uint64_t>(rows) * parts;
    if (blocks > 0x7fffffffu) return fail(TH_KERNEL_ERROR, "rms_norm: grid too large");
    void* stv = nullptr;
    TH_TRY(th::stream_scratch(s, blocks * sizeof(float), &stv));
    auto* st = static_cast<float*>(stv);
    const dim3 grid(static_cast<uint32_t>(blocks)), block(256);
    const uint32_t P = static_cast<uint32_t>(parts), Cn = static_cast<uint32_t>(chunk);
    hipLaunchKernelGGL((th::rms_norm_part_stats<DT>), grid, block, 0, s, x, st, cols, P, Cn);
    if (same_phase16(x, y))
      hipLaunchKernelGGL((th::rms_norm_part_apply<DT, true>), grid, block, 0, s, x, y, st, cols, P,
                         Cn, eps);
    else
      hipLaunchKernelGGL((th::rms_norm_part_apply<DT, false>), grid, block, 0, s, x, y, st, cols,
                         P, Cn, eps);
  }
  return launch_status("rms_norm launch");
}

// ---- random fill ------------------------------------------------------------------

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

template <int DT>
__global__ void __launch_bounds__(256)
fill_random_kernel(void* dst, uint64_t n, int dist, float p0, float p1, uint64_t seed) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const uint64_t r = splitmix64(seed ^ splitmix64(i));
  const float u1 = (static_cast<float>(r >> 40) + 0.5f) * (1.0f / 16777216.0f);           // (0,1)
  const float u2 = static_cast<float>((r >> 16) & 0xffffffu) * (1.0f / 16777216.0f);     // [0,1)
  float v;
  if (dist == 0) {
    v = p0 + (p1 - p0) * u2;
  } else {
    v = p0 + p1 * sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
  }
  if constexpr (DT == th::kF32) static_cast<float*>(dst)[i] = v;
  else static_cast<uint16_t*>(dst)[i] = th::f32_to_u16<DT>(v);
}

}  // namespace

extern "C" {

int th_softmax(const void* x, void* y, uint32_t rows, uint32_t cols, th_dtype dtype, th_stream s) {
  if (!valid_dtype(dtype)) return fail(TH_KERNEL_ERROR, "softmax: unknown dtype");
  if (rows == 0 || cols == 0) return TH_OK;
  if (!x || !y) return fail(TH_KERNEL_ERROR, "softmax: null pointer");
  switch (dtype) {
    case TH_F32: return softmax_launch<th::kF32>(x, y, rows, cols, as_stream(s));
    case TH_F16: return softmax_launch<th::kF16>(x, y, rows, cols, as_stream(s));
    default: return softmax_launch<th::kBF16>(x, y, rows, cols, as_stream(s));
  }
}

int th_rms_norm(const void* x, void* y, uint32_t rows, uint32_t cols, float eps, th_dtype dtype,
                th_stream s) {
  if (!valid_dtype(dtype)) return fail(TH_KERNEL_ERROR, "rms_norm: unknown dtype");
  if (rows == 0 || cols == 0) return TH_OK;
  if (!x || !y) return fail(TH_KERNEL_ERROR, "rms_norm: null pointer");
  if (!(eps >= 0.0f)) return fail(TH_KERNEL_ERROR, "rms_norm: eps must be >= 0");
  switch (dtype) {
    case TH_F32: return rms_norm_launch<th::kF32>(x, y, rows, cols, eps, as_stream(s));
    case TH_F16: return rms_norm_launch<th::kF16>(x, y, rows, cols, eps, as_stream(s));
    default: return rms_norm_launch<th::kBF16>(x, y, rows, cols, eps, as_stream(s));
  }
}

int th_causal_mask_f32(const float* x, float* y, uint32_t rows, uint32_t cols, uint32_t tiles,
                       th_stream s) {
  const uint64_t total = static_cast<uint64_t>(rows) * cols * tiles;
  if (total == 0) return TH_OK;
  if (!x || !y) return fail(TH_KERNEL_ERROR, "causal_mask: null pointer");
  const uint64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffffu) return fail(TH_KERNEL_ERROR, "causal_mask: too large");
  hipLaunchKernelGGL(th::causal_mask_f32, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                     as_stream(s), x, y, rows, cols, total);
  return launch_status("causal_mask launch");
}

static int attn_general_launch(const void* q, const void* k, const void* v, void* o,
                               uint32_t batch, uint32_t seq_len, uint32_t start_pos,
                               uint32_t max_seq, uint32_t kv_len, uint32_t head_dim, uint32_t nh,
                               uint32_t nkv, int causal, float scale, th_dtype dtype,
                               hipStream_t s) {
  if (head_dim > 256) return fail(TH_KERNEL_ERROR, "attention: head_dim > 256 is not supported");
  const uint64_t blocks = static_cast<uint64_t>(batch) * seq_len * nh;
  if (blocks > 0x7fffffffu) return fail(TH_KERNEL_ERROR, "attention: grid too large");
  const dim3 grid(static_cast<uint32_t>(blocks)), block(256);
  switch (dtype) {
    case TH_F32:
      hipLaunchKernelGGL(th::attn_general<th::kF32>, grid, block, 0, s, q, k, v, o, batch, seq_len,
                         start_pos, max_seq, kv_len, head_dim, nh, nkv, causal, scale);
      break;
    case TH_F16:
      hipLaunchKernelGGL(th::attn_general<th::kF16>, grid, block, 0, s, q, k, v, o, batch, seq_len,
                         start_pos, max_seq, kv_len, head_dim, nh, nkv, causal, scale);
      break;
    default:
      hipLaunchKernelGGL(th::attn_general<th::kBF16>, grid, block, 0, s, q, k, v, o, batch,
                         seq_len, start_pos, max_seq, kv_len, head_dim, nh, nkv, causal, scale);
      break;
  }
  return launch_status("attention (general) launch");
}

int th_attention(const void* q, const void* k, const void* v, void* o, uint32_t seq_len,
                 uint32_t head_dim, uint32_t tiles, th_dtype dtype, th_stream s) {
  if (!valid_dtype(dtype)) return fail(TH_KERNEL_ERROR, "attention: unknown dtype");
  if (seq_len == 0 || head_dim == 0 || tiles == 0) return TH_OK;
  if (!q || !k || !v || !o) return fail(TH_KERNEL_ERROR, "attention: null pointer");
  // scale printed by the linalg bridge: 1.0f64 / sqrt(d), then used as f32
  const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(head_dim)));
  if (dtype == TH_F32 && (head_dim == 64 || head_dim == 128) && aligned16(q) && aligned16(k) &&
      aligned16(v)) {
    // the fp32 MFMA flash kernel: one workgroup per (tile, 128 queries)
    const uint64_t blocks = static_cast<uint64_t>(tiles) * ((seq_len + th::af32::BQ - 1) / th::af32::BQ);
    if (blocks > 0x7fffffffu) return fail(TH_KERNEL_ERROR, "attention: too many tiles");
    const dim3 grid(static_cast<uint32_t>(blocks)), block(th::af32::NT);
    auto Q = static_cast<const float*>(q);
    auto K = static_cast<const float*>(k);
    auto V = static_cast<const float*>(v);
    auto O = static_cast<float*>(o);
    if (head_dim == 64)
      hipLaunchKernelGGL(th::attn_f32_mfma<64>, grid, block, 0, as_stream(s), Q, K, V, O, seq_len,
                         scale * th::kLog2e);
    else
      hipLaunchKernelGGL(th::attn_f32_mfma<128>, grid, block, 0, as_stream(s), Q, K, V, O,
                         seq_len, scale * th::kLog2e);
    return launch_status("attention (fp32 MFMA) launch");
  }
  return attn_general_launch(q, k, v, o, tiles, seq_len, 0, seq_len, seq_len, head_dim, 1, 1, 0,
                             scale, dtype, as_stream(s));
}

// Copy rows of 16-bit values in 16-byte pieces.  Destination row i (of `rows`)
// is source row (i / grp) * src_grp + i % grp: the first `grp` rows of every
// group of `src_grp` source rows.  Each row takes the first cols8 pieces of the
// source row (src_ld8 pieces long) and zeros up to dst_ld8 pieces.
__global__ void __launch_bounds__(256)
copy_rows16(const uint4* __restrict__ src, uint32_t src_ld8, uint4* __restrict__ dst,
            uint32_t dst_ld8, uint32_t cols8, uint64_t rows, uint32_t grp, uint32_t src_grp) {
  const uint64_t n = rows * dst_ld8;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x; i < n;
       i += static_cast<uint64_t>(gridDim.x) * 256u) {
    const uint64_t r = i / dst_ld8;
    const uint64_t sr = (r / grp) * src_grp + r % grp;
    const uint32_t c = static_cast<uint32_t>(i % dst_ld8);
    dst[i] = c < cols8 ? src[sr * src_ld8 + c] : make_uint4(0, 0, 0, 0);
  }
}

static void copy_rows16_launch(const void* src, uint32_t src_ld, void* dst, uint32_t dst_ld,
                               uint32_t cols, uint64_t rows, hipStream_t s, uint32_t grp = 0,
                               uint32_t src_grp = 0) {
  const uint64_t n = rows * (dst_ld / 8);
  const uint32_t blocks =
      static_cast<uint32_t>(std::min<uint64_t>((n + 255) / 256, 8ull * current_cu_count()));
  if (grp == 0) grp = src_grp = 0xffffffffu;  // plain: row i <- row i
  hipLaunchKernelGGL(copy_rows16, dim3(std::max(blocks, 1u)), dim3(256), 0, s,
                     static_cast<const uint4*>(src), src_ld / 8, static_cast<uint4*>(dst),
                     dst_ld / 8, cols / 8, rows, grp, src_grp);
}

}  // extern "C"

// The prefill kernels for head dim HD: one pass, or (nsplit > 1) split-KV parts and
// their merge.
template <int HD>
static void prefill_launch(th_dtype dtype, const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                           uint16_t* O, float* part_ws, uint32_t batch, uint32_t seq_len,
                           uint32_t start_pos, uint32_t kv_rows, uint32_t nh, uint32_t nkv,
                           float sl2, uint64_t blocks, uint64_t rows_q, uint32_t nsplit,
                           uint32_t chunk, hipStream_t s) {
  const dim3 block(th::pfa::NT);
  if (nsplit > 1) {
    constexpr uint32_t rpb = 256 / (HD / 4);   // rows per merge workgroup
    const dim3 sgrid(static_cast<uint32_t>(blocks * nsplit));
    const dim3 cgrid(static_cast<uint32_t>((rows_q + rpb - 1) / rpb));
    if (dtype == TH_BF16) {
      hipLaunchKernelGGL((th::pfa::attn_prefill_split<th::kBF16, HD>), sgrid, block, 0, s, Q, K, V,
                         part_ws, batch, seq_len, start_pos, kv_rows, nh, nkv, sl2, nsplit, chunk);
      hipLaunchKernelGGL((th::pfa::attn_prefill_combine<th::kBF16, HD>), cgrid, dim3(256), 0, s,
                         part_ws, O, static_cast<size_t>(rows_q), nsplit);
    } else {
      hipLaunchKernelGGL((th::pfa::attn_prefill_split<th::kF16, HD>), sgrid, block, 0, s, Q, K, V,
                         part_ws, batch, seq_len, start_pos, kv_rows, nh, nkv, sl2, nsplit, chunk);
      hipLaunchKernelGGL((th::pfa::attn_prefill_combine<th::kF16, HD>), cgrid, dim3(256), 0, s,
                         part_ws, O, static_cast<size_t>(rows_q), nsplit);
    }
    return;
  }
  const dim3 grid(static_cast<uint32_t>(blocks));
  if (dtype == TH_BF16)
    hipLaunchKernelGGL((th::pfa::attn_prefill_asm<th::kBF16, HD>), grid, block, 0, s, Q, K, V, O,
                       batch, seq_len, start_pos, kv_rows, nh, nkv, sl2);
  else
    hipLaunchKernelGGL((th::pfa::attn_prefill_asm<th::kF16, HD>), grid, block, 0, s, Q, K, V, O,
                       batch, seq_len, start_pos, kv_rows, nh, nkv, sl2);
}

extern "C" {

int th_attention_prefill(const void* q, const void* k, const void* v, void* o, uint32_t batch,
                         uint32_t seq_len, uint32_t start_pos, uint32_t max_seq,
                         uint32_t head_dim, uint32_t num_heads, uint32_t num_kv_heads,
                         th_dtype dtype, th_stream s) {
  if (!valid_dtype(dtype)) return fail(TH_KERNEL_ERROR, "attention_prefill: unknown dtype");
  if (batch == 0 || seq_len == 0 || num_heads == 0) return TH_OK;
  if (!q || !k || !v || !o) return fail(TH_KERNEL_ERROR, "attention_prefill: null pointer");
  if (num_kv_heads == 0 || num_heads % num_kv_heads != 0)
    return fail(TH_KERNEL_ERROR, "attention_prefill: num_heads must be a multiple of num_kv_heads");
  if (static_cast<uint64_t>(start_pos) + seq_len > max_seq)
    return fail(TH_KERNEL_ERROR, "attention_prefill: start_pos + seq_len exceeds max_seq");
  if (head_dim == 0) return fail(TH_KERNEL_ERROR, "attention_prefill: head_dim == 0");
  const float scale = 1.0f / std::sqrt(static_cast<float>(head_dim));  // rsqrt(float(head_dim))
  const bool vec16 = aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o);
  // head_dim 128 and 64 run natively
  const bool fast = dtype != TH_F32 && (head_dim == th::pfa::D || head_dim == 64) && vec16;
  // Head dims below 128 (multiples of 8) run the same kernel on copies zero-padded
  // to 128 columns: the zero columns add nothing to Q.K^T and give zero O columns,
  // so the result is that of the narrower head (with its own 1/sqrt(D) scale).
  // Half the MFMA work is padding, against a general kernel ~500x slower
  // (measured for D = 64, S = 2048-4096).
  const bool pad = !fast && dtype != TH_F32 && head_dim < th::pfa::D && head_dim % 8 == 0 && vec16;
  const uint32_t hd = fast ? head_dim : th::pfa::D;   // the kernel's head dim
  if (fast || pad) {
    const uint64_t nqb = (seq_len + th::pfa::BQ - 1) / th::pfa::BQ;
    const uint64_t blocks = nqb * batch * num_heads;
    if (blocks > 0x7fffffffu) return fail(TH_KERNEL_ERROR, "attention_prefill: grid too large");
    const float sl2 = scale * th::kLog2e;
    auto Q = static_cast<const uint16_t*>(q);
    auto K = static_cast<const uint16_t*>(k);
    auto V = static_cast<const uint16_t*>(v);
    auto O = static_cast<uint16_t*>(o);
    uint32_t kv_rows = max_seq;   // cache rows per (batch, kv head) seen by the kernel
    const uint64_t rows_q = static_cast<uint64_t>(batch) * seq_len * num_heads;
    // Split-KV: too few work items to fill the chip (a short chunk after a long cache)
    // split each item's cached blocks below start_pos into parts whose partial (O, l, m)
    // rows a second kernel merges.  Each part keeps >= 8 cached blocks; every part but the
    // last starts and ends below start_pos, so every row of a part has unmasked keys.
    const uint32_t cus = current_cu_count();
    const uint32_t cached = start_pos / th::pfa::BKV;
    uint32_t nsplit = 1, chunk = 0;
    if (blocks < cus && cached >= 16) {
      nsplit = static_cast<uint32_t>(std::min<uint64_t>((cus + blocks - 1) / blocks, cached / 8));
      nsplit = std::min<uint32_t>(nsplit, 16);
      if (nsplit >= 2) {
        const uint32_t nb_max = (start_pos + seq_len + th::pfa::BKV - 1) / th::pfa::BKV;
        chunk = std::min((nb_max + nsplit - 1) / nsplit, cached / (nsplit - 1));
      } else {
        nsplit = 1;
      }
    }
    const uint64_t split_bytes =
        nsplit > 1 ? static_cast<uint64_t>(nsplit) * rows_q * th::pfa::part_rec(hd) * 4 : 0;
    float* part_ws = nullptr;
    if (split_bytes && !pad) {
      void* ws = nullptr;
      TH_TRY(th::stream_scratch(as_stream(s), split_bytes, &ws));
      part_ws = static_cast<float*>(ws);
    }
    if (pad) {
      // Only the live cache rows (positions < start_pos + seq_len) are read, so only
      // those are copied: the padded cache holds kv_len rows per (batch, kv head).
      const uint32_t kv_len = start_pos + seq_len;
      const uint64_t rows_kv = static_cast<uint64_t>(batch) * num_kv_heads * kv_len;
      constexpr uint64_t RB = th::pfa::D * 2;  // bytes of a padded row
      void* ws = nullptr;
      const uint64_t pad_bytes = (2 * rows_q + 2 * rows_kv) * RB;
      TH_TRY(th::stream_scratch(as_stream(s), pad_bytes + split_bytes, &ws));
      auto* base = static_cast<uint16_t*>(ws);
      if (split_bytes) part_ws = reinterpret_cast<float*>(static_cast<char*>(ws) + pad_bytes);
      uint16_t* Qp = base;
      uint16_t* Op = Qp + rows_q * th::pfa::D;
      uint16_t* Kp = Op + rows_q * th::pfa::D;
      uint16_t* Vp = Kp + rows_kv * th::pfa::D;
      copy_rows16_launch(q, head_dim, Qp, th::pfa::D, head_dim, rows_q, as_stream(s));
      copy_rows16_launch(k, head_dim, Kp, th::pfa::D, head_dim, rows_kv, as_stream(s), kv_len,
                         max_seq);
      copy_rows16_launch(v, head_dim, Vp, th::pfa::D, head_dim, rows_kv, as_stream(s), kv_len,
                         max_seq);
      TH_TRY(launch_status("attention_prefill padding"));
      Q = Qp;
      K = Kp;
      V = Vp;
      O = Op;
      kv_rows = kv_len;
    }
    if (hd == 64)
      prefill_launch<64>(dtype, Q, K, V, O, part_ws, batch, seq_len, start_pos, kv_rows, num_heads,
                         num_kv_heads, sl2, blocks, rows_q, nsplit, chunk, as_stream(s));
    else
      prefill_launch<th::pfa::D>(dtype, Q, K, V, O, part_ws, batch, seq_len, start_pos, kv_rows,
                                 num_heads, num_kv_heads, sl2, blocks, rows_q, nsplit, chunk,
                                 as_stream(s));
    TH_TRY(launch_status("attention_prefill launch"));
    if (pad) {
      copy_rows16_launch(O, th::pfa::D, o, head_dim, head_dim, rows_q, as_stream(s));
      return launch_status("attention_prefill unpadding");
    }
    return TH_OK;
  }
  return attn_general_launch(q, k, v, o, batch, seq_len, start_pos, max_seq, start_pos + seq_len,
                             head_dim, num_heads, num_kv_heads, 1, scale, dtype, as_stream(s));
}

static uint32_t decode_chunks(uint32_t seq_len) {
  return (seq_len + th::dec::CHUNK - 1) / th::dec::CHUNK;
}

// KV split of the decode: about two workgroups per CU in total (measured on
// MI355X: config 5's 512 (batch, kv_head) items run fastest unsplit, 332 us
// against 350 us with one workgroup per chunk; a single item at 32K positions
// wants 64 splits), then chunks spread evenly so that no split is empty.
static void decode_plan(uint32_t items, uint32_t nchunks, uint32_t* n_split, uint32_t* cps) {
  const uint32_t target = 2 * current_cu_count();
  uint32_t n = (target + items - 1) / items;
  n = std::max(1u, std::min(n, nchunks));
  *cps = (nchunks + n - 1) / n;
  *n_split = (nchunks + *cps - 1) / *cps;
}

// The MFMA decode: head_dim 128 or 64 (both native), G = 1..16 query heads per kv head.
static bool decode_fast(uint32_t head_dim, uint32_t nh, uint32_t nkv, th_dtype dtype) {
  if (dtype == TH_F32 || (head_dim != th::dec::D && head_dim != 64) || nkv == 0 || nh % nkv != 0)
    return false;
  const uint32_t g = nh / nkv;
  return g == 1 || g == 2 || g == 4 || g == 8 || g == 16;
}

size_t th_attention_decode_workspace_size(uint32_t batch, uint32_t seq_len, uint32_t head_dim,
                                          uint32_t num_heads, uint32_t num_kv_heads) {
  (void)num_kv_heads;
  // 128 and 64 run natively; other head dims below 128 (multiples of 8) run the
  // 128-wide kernel on padded copies.  Records are sized for 128 columns either way.
  if (head_dim > th::dec::D || head_dim == 0 || (head_dim != th::dec::D && head_dim % 8 != 0))
    return 0;
  return static_cast<size_t>(batch) * num_heads * decode_chunks(seq_len) * (th::dec::D + 2) *
         sizeof(float);
}

}  // extern "C"

template <int DT, int G, int HD>
static void decode_split_launch(const void* q, const void* k, const void* v, void* o, float* ws,
                                uint32_t batch, uint32_t seq_len, uint32_t max_seq, uint32_t nh,
                                uint32_t nkv, uint32_t n_split, uint32_t cps, float sl2,
                                hipStream_t s) {
  const dim3 grid(batch * nkv * n_split), block(th::dec::NT);
  hipLaunchKernelGGL((th::attn_decode_split<DT, G, HD>), grid, block, 0, s,
                     static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                     static_cast<const uint16_t*>(v), static_cast<uint16_t*>(o), ws, seq_len,
                     max_seq, nh, nkv, n_split, cps, sl2);
}

template <int DT, int HD>
static void decode_launch_g(uint32_t g, const void* q, const void* k, const void* v, void* o,
                            float* ws, uint32_t batch, uint32_t seq_len, uint32_t max_seq,
                            uint32_t nh, uint32_t nkv, uint32_t n_split, uint32_t cps, float sl2,
                            hipStream_t s) {
  switch (g) {
    case 1: decode_split_launch<DT, 1, HD>(q, k, v, o, ws, batch, seq_len, max_seq, nh, nkv, n_split, cps, sl2, s); break;
    case 2: decode_split_launch<DT, 2, HD>(q, k, v, o, ws, batch, seq_len, max_seq, nh, nkv, n_split, cps, sl2, s); break;
    case 4: decode_split_launch<DT, 4, HD>(q, k, v, o, ws, batch, seq_len, max_seq, nh, nkv, n_split, cps, sl2, s); break;
    case 8: decode_split_launch<DT, 8, HD>(q, k, v, o, ws, batch, seq_len, max_seq, nh, nkv, n_split, cps, sl2, s); break;
    default: decode_split_launch<DT, 16, HD>(q, k, v, o, ws, batch, seq_len, max_seq, nh, nkv, n_split, cps, sl2, s); break;
  }
}


// ---- th_attention_decode_static: the decode without any allocation ----------------
// Its split partials live in `scratch`, a fixed array in each GPU's memory that comes
// with the code object (no hipMalloc) and is held until the process ends.  Host code
// never passes the array's name to a kernel: its per-device address comes from
// hipGetSymbolAddress, looked up once per device with that device current.
constexpr size_t kDecodeStaticBytes = size_t(8) << 20;
static __device__ __align__(256) float scratch[kDecodeStaticBytes / sizeof(float)];

namespace {
std::mutex g_scratch_addr_mu;
float* g_scratch_addr[64] = {};

// bytes of the current device set to zero (the decode of an empty sequence)
__global__ void __launch_bounds__(256) zero_bytes(unsigned char* p, uint64_t n) {
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x; i < n;
       i += static_cast<uint64_t>(gridDim.x) * 256u)
    p[i] = 0;
}
}  // namespace

static int static_scratch_address(float** out) {
  int dev = 0;
  TH_TRY(th::check_hip(hipGetDevice(&dev), "hipGetDevice", TH_DEVICE_ERROR));
  if (dev < 0 || dev >= 64) return fail(TH_DEVICE_ERROR, "attention_decode_static: device ordinal >= 64");
  std::lock_guard<std::mutex> lock(g_scratch_addr_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    TH_TRY(th::check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress",
                         TH_MEMORY_ERROR));
    if (!p) return fail(TH_MEMORY_ERROR, "attention_decode_static: no address for the scratch array");
    g_scratch_addr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_addr[dev];
  return TH_OK;
}

// The MFMA decode (head_dim 128 or 64): split kernel, then (n_split > 1) the LSE
// combine of the partials in ws.  Launches only; no allocation.
template <int HD>
static void decode_run_hd(const void* Q, const void* K, const void* V, void* O, float* ws,
                          uint32_t batch, uint32_t seq_len, uint32_t max_seq, uint32_t num_heads,
                          uint32_t num_kv_heads, uint32_t n_split, uint32_t cps, float sl2,
                          th_dtype dtype, hipStream_t s) {
  const uint32_t g = num_heads / num_kv_heads;
  if (dtype == TH_BF16)
    decode_launch_g<th::kBF16, HD>(g, Q, K, V, O, ws, batch, seq_len, max_seq, num_heads,
                                   num_kv_heads, n_split, cps, sl2, s);
  else
    decode_launch_g<th::kF16, HD>(g, Q, K, V, O, ws, batch, seq_len, max_seq, num_heads,
                                  num_kv_heads, n_split, cps, sl2, s);
  // with one split each workgroup covered its whole sequence and wrote O
  if (n_split > 1) {
    const dim3 cgrid(batch * num_heads), cblock(th::dec::CT);
    if (dtype == TH_BF16)
      hipLaunchKernelGGL((th::attn_decode_combine<th::kBF16, HD>), cgrid, cblock, 0, s, ws,
                         static_cast<uint16_t*>(O), num_heads, num_kv_heads, n_split);
    else
      hipLaunchKernelGGL((th::attn_decode_combine<th::kF16, HD>), cgrid, cblock, 0, s, ws,
                         static_cast<uint16_t*>(O), num_heads, num_kv_heads, n_split);
  }
}

static int decode_run(const void* Q, const void* K, const void* V, void* O, float* ws,
                      uint32_t batch, uint32_t seq_len, uint32_t max_seq, uint32_t head_dim,
                      uint32_t num_heads, uint32_t num_kv_heads, uint32_t n_split, uint32_t cps,
                      float sl2, th_dtype dtype, hipStream_t s) {
  if (head_dim == 64)
    decode_run_hd<64>(Q, K, V, O, ws, batch, seq_len, max_seq, num_heads, num_kv_heads, n_split,
                      cps, sl2, dtype, s);
  else
    decode_run_hd<th::dec::D>(Q, K, V, O, ws, batch, seq_len, max_seq, num_heads, num_kv_heads,
                              n_split, cps, sl2, dtype, s);
  return launch_status("attention_decode launch");
}

extern "C" {

// The shapes th_attention_decode runs on zero-padded 128-column copies (when the
// native MFMA decode does not take them): 16-bit head dims below 128 that are
// multiples of 8, with a group size the MFMA decode takes and 16-byte aligned views.
static bool decode_pad(const void* q, const void* k, const void* v, const void* o,
                       uint32_t head_dim, uint32_t num_heads, uint32_t num_kv_heads,
                       th_dtype dtype) {
  return head_dim < th::dec::D && head_dim % 8 == 0 &&
         decode_fast(th::dec::D, num_heads, num_kv_heads, dtype) && aligned16(q) &&
         aligned16(k) && aligned16(v) && aligned16(o);
}

int th_attention_decode(const void* q, const void* k, const void* v, void* o, uint32_t batch,
                        uint32_t seq_len, uint32_t max_seq, uint32_t head_dim, uint32_t num_heads,
                        uint32_t num_kv_heads, th_dtype dtype, void* workspace,
                        size_t workspace_bytes, th_stream s) {
  if (!valid_dtype(dtype)) return fail(TH_KERNEL_ERROR, "attention_decode: unknown dtype");
  if (batch == 0 || num_heads == 0) return TH_OK;
  if (!q || !k || !v || !o) return fail(TH_KERNEL_ERROR, "attention_decode: null pointer");
  if (num_kv_heads == 0 || num_heads % num_kv_heads != 0)
    return fail(TH_KERNEL_ERROR, "attention_decode: num_heads must be a multiple of num_kv_heads");
  if (seq_len > max_seq) return fail(TH_KERNEL_ERROR, "attention_decode: seq_len exceeds max_seq");
  if (head_dim == 0) return fail(TH_KERNEL_ERROR, "attention_decode: head_dim == 0");
  const float scale = 1.0f / std::sqrt(static_cast<float>(head_dim));
  if (seq_len == 0) {
    // no positions: the output is zero (nothing to weight)
    const size_t bytes = static_cast<size_t>(batch) * num_heads * head_dim * dtype_size(dtype);
    return th::check_hip(hipMemsetAsync(o, 0, bytes, as_stream(s)), "hipMemsetAsync",
                         TH_MEMORY_ERROR);
  }
  const bool fast = decode_fast(head_dim, num_heads, num_kv_heads, dtype) && aligned16(q) &&
                    aligned16(k) && aligned16(v);
  // Other head dims below 128 (multiples of 8): Q and the live rows of K and V (the first
  // seq_len of each (batch, kv_head)) are copied zero-padded to 128 columns into the
  // stream's scratch, the MFMA decode runs on the copies (zero columns change no
  // score and give zero outputs) and O's first head_dim columns are copied back.
  // The split partials use the caller's workspace as for head_dim 128.  The copies
  // read K and V once more, but the general kernel is 20-70x slower (measured for
  // head_dim 64).
  const bool pad = !fast && decode_pad(q, k, v, o, head_dim, num_heads, num_kv_heads, dtype);
  if (!fast && !pad) {
    // one query per (batch, head): Q/O [B][1][NH][D]
    return attn_general_launch(q, k, v, o, batch, 1, 0, max_seq, seq_len, head_dim, num_heads,
                               num_kv_heads, 0, scale, dtype, as_stream(s));
  }
  const void* Q = q;
  const void* K = k;
  const void* V = v;
  void* O = o;
  if (pad) {
    constexpr uint64_t RB = th::dec::D * 2;
    const uint64_t rows_q = static_cast<uint64_t>(batch) * num_heads;
    const uint64_t rows_kv = static_cast<uint64_t>(batch) * num_kv_heads * seq_len;
    void* pw = nullptr;
    TH_TRY(th::stream_scratch(as_stream(s), (2 * rows_q + 2 * rows_kv) * RB, &pw));
    auto* base = static_cast<uint16_t*>(pw);
    uint16_t* Qp = base;
    uint16_t* Op = Qp + rows_q * th::dec::D;
    uint16_t* Kp = Op + rows_q * th::dec::D;
    uint16_t* Vp = Kp + rows_kv * th::dec::D;
    copy_rows16_launch(q, head_dim, Qp, th::dec::D, head_dim, rows_q, as_stream(s));
    copy_rows16_launch(k, head_dim, Kp, th::dec::D, head_dim, rows_kv, as_stream(s), seq_len,
                       max_seq);
    copy_rows16_launch(v, head_dim, Vp, th::dec::D, head_dim, rows_kv, as_stream(s), seq_len,
                       max_seq);
    TH_TRY(launch_status("attention_decode padding"));
    Q = Qp;
    K = Kp;
    V = Vp;
    O = Op;
    max_seq = seq_len;  // the copies hold the live rows only
  }
  const uint64_t items = static_cast<uint64_t>(batch) * num_kv_heads;
  if (items > 0x7fffffffu) return fail(TH_KERNEL_ERROR, "attention_decode: grid too large");
  uint32_t n_split, cps;
  decode_plan(static_cast<uint32_t>(items), decode_chunks(seq_len), &n_split, &cps);
  const uint64_t blocks = items * n_split;
  if (blocks > 0x7fffffffu) return fail(TH_KERNEL_ERROR, "attention_decode: grid too large");
  // The workspace contract does not depend on the split chosen here: callers
  // size it with th_attention_decode_workspace_size (one record per chunk).
  const size_t need = th_attention_decode_workspace_size(batch, seq_len, th::dec::D, num_heads,
                                                         num_kv_heads);
  void* ws = workspace;
  if (ws) {
    if (workspace_bytes < need)
      return fail(TH_MEMORY_ERROR, "attention_decode: workspace of " +
                                       std::to_string(workspace_bytes) + " bytes < required " +
                                       std::to_string(need));
  } else if (n_split > 1) {
    TH_TRY(th::device_scratch(need, &ws));
  }
  TH_TRY(decode_run(Q, K, V, O, static_cast<float*>(ws), batch, seq_len, max_seq,
                    pad ? th::dec::D : head_dim, num_heads, num_kv_heads, n_split, cps,
                    scale * th::kLog2e, dtype, as_stream(s)));
  if (pad) {
    copy_rows16_launch(O, th::dec::D, o, head_dim, head_dim,
                       static_cast<uint64_t>(batch) * num_heads, as_stream(s));
    return launch_status("attention_decode unpadding");
  }
  return TH_OK;
}

int th_attention_decode_static(const void* q, const void* k, const void* v, void* o,
                               uint32_t batch, uint32_t seq_len, uint32_t max_seq,
                               uint32_t head_dim, uint32_t num_heads, uint32_t num_kv_heads,
                               th_dtype dtype, th_stream s) {
  if (!valid_dtype(dtype)) return fail(TH_KERNEL_ERROR, "attention_decode_static: unknown dtype");
  if (batch == 0 || num_heads == 0) return TH_OK;
  if (!q || !k || !v || !o) return fail(TH_KERNEL_ERROR, "attention_decode_static: null pointer");
  if (num_kv_heads == 0 || num_heads % num_kv_heads != 0)
    return fail(TH_KERNEL_ERROR,
                "attention_decode_static: num_heads must be a multiple of num_kv_heads");
  if (seq_len > max_seq)
    return fail(TH_KERNEL_ERROR, "attention_decode_static: seq_len exceeds max_seq");
  if (head_dim == 0) return fail(TH_KERNEL_ERROR, "attention_decode_static: head_dim == 0");
  const float scale = 1.0f / std::sqrt(static_cast<float>(head_dim));
  if (seq_len == 0) {
    const uint64_t bytes = static_cast<uint64_t>(batch) * num_heads * head_dim * dtype_size(dtype);
    const uint32_t blocks =
        static_cast<uint32_t>(std::min<uint64_t>((bytes + 255) / 256, 4ull * current_cu_count()));
    hipLaunchKernelGGL(zero_bytes, dim3(std::max(blocks, 1u)), dim3(256), 0, as_stream(s),
                       static_cast<unsigned char*>(o), bytes);
    return launch_status("attention_decode_static zero");
  }
  const bool fast = decode_fast(head_dim, num_heads, num_kv_heads, dtype) && aligned16(q) &&
                    aligned16(k) && aligned16(v);
  if (!fast) {
    // th_attention_decode would pad these shapes into allocated copies; every other
    // shape it runs on the general kernel, which needs no scratch
    if (decode_pad(q, k, v, o, head_dim, num_heads, num_kv_heads, dtype))
      return fail(TH_KERNEL_ERROR,
                  "attention_decode_static: head_dim " + std::to_string(head_dim) +
                      " runs on zero-padded copies that need allocated memory; use "
                      "th_attention_decode");
    // the general kernel needs no scratch
    return attn_general_launch(q, k, v, o, batch, 1, 0, max_seq, seq_len, head_dim, num_heads,
                               num_kv_heads, 0, scale, dtype, as_stream(s));
  }
  const uint64_t items = static_cast<uint64_t>(batch) * num_kv_heads;
  if (items > 0x7fffffffu) return fail(TH_KERNEL_ERROR, "attention_decode_static: grid too large");
  uint32_t n_split, cps;
  decode_plan(static_cast<uint32_t>(items), decode_chunks(seq_len), &n_split, &cps);
  if (items * n_split > 0x7fffffffu)
    return fail(TH_KERNEL_ERROR, "attention_decode_static: grid too large");
  float* ws = nullptr;
  if (n_split > 1) {
    const uint64_t need =
        static_cast<uint64_t>(batch) * num_heads * n_split * (head_dim + 2) * sizeof(float);
    if (need > kDecodeStaticBytes)
      return fail(TH_MEMORY_ERROR, "attention_decode_static: the split partials need " +
                                       std::to_string(need) + " bytes, more than the " +
                                       std::to_string(kDecodeStaticBytes) +
                                       "-byte fixed scratch; use th_attention_decode");
    TH_TRY(static_scratch_address(&ws));
  }
  return decode_run(q, k, v, o, ws, batch, seq_len, max_seq, head_dim, num_heads, num_kv_heads,
                    n_split, cps, scale * th::kLog2e, dtype, as_stream(s));
}

int th_fill_random(void* dst, uint64_t n, th_dtype dtype, int dist, float p0, float p1,
                   uint64_t seed, th_stream s) {
  if (!valid_dtype(dtype)) return fail(TH_KERNEL_ERROR, "fill_random: unknown dtype");
  if (dist != 0 && dist != 1) return fail(TH_KERNEL_ERROR, "fill_random: dist must be 0 or 1");
  if (n == 0) return TH_OK;
  if (!dst) return fail(TH_KERNEL_ERROR, "fill_random: null pointer");
  const uint64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffffu) return fail(TH_KERNEL_ERROR, "fill_random: too large");
  const dim3 grid(static_cast<uint32_t>(blocks)), block(256);
  switch (dtype) {
    case TH_F32:
      hipLaunchKernelGGL(fill_random_kernel<th::kF32>, grid, block, 0, as_stream(s), dst, n, dist, p0,
                         p1, seed);
      break;
    case TH_F16:
      hipLaunchKernelGGL(fill_random_kernel<th::kF16>, grid, block, 0, as_stream(s), dst, n, dist, p0,
                         p1, seed);
      break;
    default:
      hipLaunchKernelGGL(fill_random_kernel<th::kBF16>, grid, block, 0, as_stream(s), dst, n, dist,
                         p0, p1, seed);
      break;
  }
  return launch_status("fill_random launch");
}

}  // extern "C"

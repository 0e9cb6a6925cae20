// GEMM entry points of the C ABI (include/tilers_hip.h, section 2): th_matmul and
// th_matmul_silu_mul.  Shapes and pointers are checked on the host, the hand-written
// gfx950 kernel for the shape is picked and enqueued on the caller's stream; there is
// no CPU fallback.  (Its own translation unit: the GEMM instantiations compile in
// parallel with the rest of the library.)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "kernels/common.hpp"
#include "kernels/gemm.hpp"
#include "kernels/gemm_asm.hpp"
#include "kernels/gemm_f32.hpp"
#include "ops_common.hpp"

using th::fail;
using namespace th::ops;

namespace {

// ---- matmul -------------------------------------------------------------------

// One GEMM launch: C[i] = epilogue(A[i] . B[i]) for i < batch, element strides
// sa, sb, sc; `up` (epilogue kEpiSiluMul) has C's dtype, layout and strides.
struct GemmArgs {
  const void* a;
  const void* b;
  void* c;
  const void* up;
  uint32_t m, k, n;
  bool bt;
  uint32_t batch;
  uint64_t sa, sb, sc;
  hipStream_t s;
};

// The LDS-DMA pipeline serves every shape with K % 32 == 0 unless
// TILERS_HIP_GEMM_DMA=0 (a debugging switch: the register-staged kernel then
// runs them too).
bool gemm_dma() {
  static const bool v = [] {
    const char* e = std::getenv("TILERS_HIP_GEMM_DMA");
    return !(e && std::atoi(e) == 0);
  }();
  return v;
}

// Whole-tile shapes (B row-major or stored N x K) run on the generated-assembly kernel
// (gemm_asm.hpp) unless TILERS_HIP_GEMM_ASM=0 (a debugging switch: the LDS-DMA
// kernel, which gives the same bits for the plain store, then runs them).  Read on
// every call (a getenv, next to a kernel launch), so a process can compare the two.
bool gemm_asm() {
  const char* e = std::getenv("TILERS_HIP_GEMM_ASM");
  return !(e && std::atoi(e) == 0);
}

// Split-K for shapes with too few 256 x 256 tiles to fill the chip (small M:
// decode-time projections).  S slices of K (each a multiple of 32, at least 256
// deep, S a divisor of K / 32) run as the batch dimension of the DMA kernel,
// writing f32 partials to a per-stream workspace; gemm_splitk_reduce adds them
// and applies the epilogue.  Only for batch 1.  Returns 1 for no split.
uint32_t splitk_slices(const GemmArgs& g, uint32_t tiles) {
  const uint32_t cus = current_cu_count();
  if (g.batch != 1 || 2u * tiles > cus || g.k < 512) return 1;
  const uint32_t units = g.k / th::gemm::DBK;             // K in 32-deep steps
  const uint32_t cap = std::min<uint32_t>({cus / tiles, g.k / 256u, 32u});
  uint32_t best = 1;
  for (uint32_t s = 2; s <= cap; ++s)
    if (units % s == 0) best = s;
  return best;
}

template <int DT, int DTO, int EPI, bool BT>
int gemm_splitk(const GemmArgs& g, uint32_t tiles, uint32_t S) {
  const uint32_t ks = g.k / S;
  const uint64_t mn = static_cast<uint64_t>(g.m) * g.n;
  void* wv = nullptr;
  TH_TRY(th::stream_scratch(g.s, S * mn * sizeof(float), &wv));
  auto* W = static_cast<float*>(wv);
  auto go = [&](auto mi) {
    constexpr int MI = decltype(mi)::value;
    hipLaunchKernelGGL((th::gemm_dma_256<DT, th::kF32, BT, th::gemm::DBK, th::gemm::NSTAGE,
                                         th::gemm::DWAVES, th::gemm::kEpiStore, MI>),
                       dim3(tiles, S), dim3(64 * th::gemm::DWAVES), 0, g.s,
                       static_cast<const uint16_t*>(g.a), static_cast<const uint16_t*>(g.b),
                       static_cast<void*>(W), g.m, g.n, ks, static_cast<uint64_t>(ks),
                       BT ? static_cast<uint64_t>(ks) : static_cast<uint64_t>(ks) * g.n, mn,
                       static_cast<const void*>(nullptr), g.k);
  };
  // rows past M are padding: compute only the 32-row blocks that hold real rows
  if (g.m <= 32) go(std::integral_constant<int, 1>{});
  else if (g.m <= 64) go(std::integral_constant<int, 2>{});
  else go(std::integral_constant<int, 4>{});
  TH_TRY(launch_status("matmul (split-K) launch"));
  const uint32_t blocks = static_cast<uint32_t>(
      std::min<uint64_t>((mn + 255) / 256, 4ull * current_cu_count()));
  hipLaunchKernelGGL((th::gemm_splitk_reduce<DTO, EPI>), dim3(blocks), dim3(256), 0, g.s, W, g.c,
                     g.up, mn, S);
  return launch_status("matmul (split-K merge) launch");
}

template <int DT, int DTO, int EPI, bool BT>
int gemm_mfma_go(const GemmArgs& g, dim3 grid) {
  auto A = static_cast<const uint16_t*>(g.a);
  auto B = static_cast<const uint16_t*>(g.b);
  // The DMA kernel's SiLU*Mul epilogue writes C and reads UP in 16-byte pieces.
  constexpr uint64_t OSZ = (DTO == th::kF32) ? 4 : 2;
  const bool out_vec = EPI != th::gemm::kEpiSiluMul ||
                       (aligned16(g.c) && aligned16(g.up) && (g.sc * OSZ) % 16 == 0 && g.n % 8 == 0);
  if (gemm_dma() && out_vec && g.k % th::gemm::DBK == 0) {
    const uint32_t S = splitk_slices(g, grid.x);
    if (S > 1) return gemm_splitk<DT, DTO, EPI, BT>(g, grid.x, S);
    if constexpr (EPI == th::gemm::kEpiStore) {
      if (gemm_asm() && th::gasm::fits(g.m, g.n, g.k, static_cast<int>(OSZ))) {
        hipLaunchKernelGGL((th::gemm_asm_256<DT, DTO, BT>), grid, dim3(th::gasm::NT), 0, g.s, A,
                           B, g.c, g.m, g.n, g.k, g.sa, g.sb, g.sc, nullptr);
        return launch_status("matmul (MFMA asm) launch");
      }
    } else if constexpr (DTO != th::kF32) {
      // SiLU*Mul with 16-bit C (UP staged through LDS: 16-byte aligned, checked above)
      if (gemm_asm() && th::gasm::fits(g.m, g.n, g.k, static_cast<int>(OSZ))) {
        hipLaunchKernelGGL((th::gemm_asm_256<DT, DTO, BT, true>), grid, dim3(th::gasm::NT), 0, g.s,
                           A, B, g.c, g.m, g.n, g.k, g.sa, g.sb, g.sc, g.up);
        return launch_status("matmul silu*mul (MFMA asm) launch");
      }
    }
    hipLaunchKernelGGL((th::gemm_dma_256<DT, DTO, BT, th::gemm::DBK, th::gemm::NSTAGE,
                                         th::gemm::DWAVES, EPI>),
                       grid, dim3(64 * th::gemm::DWAVES), 0, g.s, A, B, g.c, g.m, g.n, g.k, g.sa,
                       g.sb, g.sc, g.up, 0u);
  } else if (g.m % th::gemm::BM == 0 && g.n % th::gemm::BN == 0 && g.k % th::gemm::BK == 0) {
    hipLaunchKernelGGL((th::gemm_mfma_256<DT, DTO, BT, 2, 2, true, EPI>), grid, dim3(256), 0, g.s,
                       A, B, g.c, g.m, g.n, g.k, g.sa, g.sb, g.sc, g.up);
  } else {
    hipLaunchKernelGGL((th::gemm_mfma_256<DT, DTO, BT, 2, 2, false, EPI>), grid, dim3(256), 0, g.s,
                       A, B, g.c, g.m, g.n, g.k, g.sa, g.sb, g.sc, g.up);
  }
  return launch_status("matmul (MFMA) launch");
}

template <int DT, int DTO, int EPI>
int gemm_launch(const GemmArgs& g, bool mfma) {
  if constexpr (DT != th::kF32) {
    if (mfma) {
      const dim3 grid(((g.m + 255) / 256) * ((g.n + 255) / 256), g.batch);
      return g.bt ? gemm_mfma_go<DT, DTO, EPI, true>(g, grid)
                  : gemm_mfma_go<DT, DTO, EPI, false>(g, grid);
    }
  }
  (void)mfma;
  if constexpr (DT == th::kF32) {
    // the fp32 MFMA kernel; 16-byte loads when every row start is 16-byte aligned
    const bool vec = aligned16(g.a) && aligned16(g.b) && g.k % 4 == 0 && (g.bt || g.n % 4 == 0) &&
                     g.sa % 4 == 0 && g.sb % 4 == 0;
    const dim3 grid(((g.m + th::gf32::BM - 1) / th::gf32::BM) * ((g.n + th::gf32::BN - 1) / th::gf32::BN),
                    g.batch),
        block(th::gf32::NT);
    auto A = static_cast<const float*>(g.a);
    auto B = static_cast<const float*>(g.b);
    if (g.bt) {
      if (vec) hipLaunchKernelGGL((th::gemm_f32_mfma<DTO, true, true, EPI>), grid, block, 0, g.s, A, B, g.c, g.m, g.n, g.k, g.sa, g.sb, g.sc, g.up);
      else hipLaunchKernelGGL((th::gemm_f32_mfma<DTO, true, false, EPI>), grid, block, 0, g.s, A, B, g.c, g.m, g.n, g.k, g.sa, g.sb, g.sc, g.up);
    } else {
      if (vec) hipLaunchKernelGGL((th::gemm_f32_mfma<DTO, false, true, EPI>), grid, block, 0, g.s, A, B, g.c, g.m, g.n, g.k, g.sa, g.sb, g.sc, g.up);
      else hipLaunchKernelGGL((th::gemm_f32_mfma<DTO, false, false, EPI>), grid, block, 0, g.s, A, B, g.c, g.m, g.n, g.k, g.sa, g.sb, g.sc, g.up);
    }
    return launch_status("matmul (fp32 MFMA) launch");
  }
  const dim3 grid(((g.m + 63) / 64) * ((g.n + 63) / 64), g.batch), block(256);
  if (g.bt)
    hipLaunchKernelGGL((th::gemm_fma_64<DT, DTO, true, EPI>), grid, block, 0, g.s, g.a, g.b, g.c,
                       g.m, g.n, g.k, g.sa, g.sb, g.sc, g.up);
  else
    hipLaunchKernelGGL((th::gemm_fma_64<DT, DTO, false, EPI>), grid, block, 0, g.s, g.a, g.b, g.c,
                       g.m, g.n, g.k, g.sa, g.sb, g.sc, g.up);
  return launch_status("matmul (FMA) launch");
}

template <int EPI>
int gemm_dispatch(const GemmArgs& g, th_dtype in, th_dtype out) {
  // f32 operands have no MFMA path; 16-bit ones need K % 8 == 0, row-major B
  // N % 8 == 0 and 16-byte aligned operands and strides.
  const bool mfma = in != TH_F32 && (g.k % 8 == 0) && (g.bt || g.n % 8 == 0) && aligned16(g.a) &&
                    aligned16(g.b) && (g.sa % 8 == 0) && (g.sb % 8 == 0);
  auto by_out = [&](auto dt) {
    constexpr int DT = decltype(dt)::value;
    switch (out) {
      case TH_F32: return gemm_launch<DT, th::kF32, EPI>(g, mfma);
      case TH_F16: return gemm_launch<DT, th::kF16, EPI>(g, mfma);
      default: return gemm_launch<DT, th::kBF16, EPI>(g, mfma);
    }
  };
  switch (in) {
    case TH_F32: return by_out(std::integral_constant<int, th::kF32>{});
    case TH_F16: return by_out(std::integral_constant<int, th::kF16>{});
    default: return by_out(std::integral_constant<int, th::kBF16>{});
  }
}

}  // namespace

extern "C" {

int th_matmul(const void* a, const void* b, void* c, uint32_t m, uint32_t k, uint32_t n,
              th_dtype in_dtype, th_dtype out_dtype, int b_transposed, uint32_t batch, uint64_t sa,
              uint64_t sb, uint64_t sc, th_stream s) {
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype))
    return fail(TH_KERNEL_ERROR, "matmul: unknown dtype");
  if (m == 0 || n == 0 || batch == 0) return TH_OK;
  if (!a || !b || !c) return fail(TH_KERNEL_ERROR, "matmul: null pointer");
  if (batch > 65535) return fail(TH_KERNEL_ERROR, "matmul: batch > 65535");
  const bool bt = b_transposed != 0;
  if (sa == 0) sa = static_cast<uint64_t>(m) * k;
  if (sb == 0) sb = static_cast<uint64_t>(k) * n;
  if (sc == 0) sc = static_cast<uint64_t>(m) * n;
  if (k == 0) {
    // empty contraction: C = 0 (linalg.fill 0 with nothing accumulated)
    const size_t esz = dtype_size(out_dtype);
    for (uint32_t i = 0; i < batch; ++i)
      TH_TRY(th::check_hip(hipMemsetAsync(static_cast<char*>(c) + i * sc * esz, 0,
                                          static_cast<size_t>(m) * n * esz, as_stream(s)),
                           "hipMemsetAsync", TH_MEMORY_ERROR));
    return TH_OK;
  }
  const GemmArgs g{a, b, c, nullptr, m, k, n, bt, batch, sa, sb, sc, as_stream(s)};
  return gemm_dispatch<th::gemm::kEpiStore>(g, in_dtype, out_dtype);
}

int th_matmul_silu_mul(const void* a, const void* b, const void* up, void* c, uint32_t m,
                       uint32_t k, uint32_t n, th_dtype in_dtype, th_dtype out_dtype,
                       int b_transposed, uint32_t batch, uint64_t sa, uint64_t sb, uint64_t sc,
                       th_stream s) {
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype))
    return fail(TH_KERNEL_ERROR, "matmul_silu_mul: unknown dtype");
  if (m == 0 || n == 0 || batch == 0) return TH_OK;
  if (!a || !b || !c || !up) return fail(TH_KERNEL_ERROR, "matmul_silu_mul: null pointer");
  if (batch > 65535) return fail(TH_KERNEL_ERROR, "matmul_silu_mul: batch > 65535");
  const bool bt = b_transposed != 0;
  if (sa == 0) sa = static_cast<uint64_t>(m) * k;
  if (sb == 0) sb = static_cast<uint64_t>(k) * n;
  if (sc == 0) sc = static_cast<uint64_t>(m) * n;
  if (k == 0) {
    // silu(0) * up = 0 everywhere
    const size_t esz = dtype_size(out_dtype);
    for (uint32_t i = 0; i < batch; ++i)
      TH_TRY(th::check_hip(hipMemsetAsync(static_cast<char*>(c) + i * sc * esz, 0,
                                          static_cast<size_t>(m) * n * esz, as_stream(s)),
                           "hipMemsetAsync", TH_MEMORY_ERROR));
    return TH_OK;
  }
  const GemmArgs g{a, b, c, up, m, k, n, bt, batch, sa, sb, sc, as_stream(s)};
  return gemm_dispatch<th::gemm::kEpiSiluMul>(g, in_dtype, out_dtype);
}

}  // extern "C"

// Host helpers shared by the C-ABI translation units (ops.hip, ops_gemm.hip).
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>

#include "runtime.hpp"

namespace th {
namespace ops {

inline hipStream_t as_stream(th_stream s) { return static_cast<hipStream_t>(s); }

inline int launch_status(const char* what) {
  return th::check_hip(hipGetLastError(), what, TH_KERNEL_ERROR);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
// x and y sit at the same offset within a 16-byte block (so do their rows).
inline bool same_phase16(const void* x, const void* y) {
  return ((reinterpret_cast<uintptr_t>(x) ^ reinterpret_cast<uintptr_t>(y)) & 15u) == 0;
}

inline int dtype_size(th_dtype d) { return d == TH_F32 ? 4 : 2; }

inline bool valid_dtype(th_dtype d) { return d == TH_F32 || d == TH_F16 || d == TH_BF16; }

// Compute units of the calling thread's current device (cached per ordinal).
inline uint32_t current_cu_count() {
  static std::atomic<uint32_t> cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  uint32_t n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    n = static_cast<uint32_t>(cus);
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace ops
}  // namespace th

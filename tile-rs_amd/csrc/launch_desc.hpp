// Launch descriptor that the `hip` codegen target emits next to every tile
// kernel, as a device global named `__th_desc_<kernel>`.
//
// tile-rs launches a tile kernel on a 1-D grid of logical tiles (the
// #[tile_kernel] prelude offsets every view by block_idx * R * C,
// crates/tile_std_macros/src/lib.rs:217-266; LaunchGrid is 1-D,
// crates/tile_hal/src/kernel.rs:46-79).  A hand-written MI355X kernel wants its
// own workgroup size and may spread one tile over several workgroups (a GEMM
// tile) or pack several tiles into one workgroup (one softmax row per wave).
// The descriptor tells the runtime how to turn the caller's tile count into the
// hardware grid; the kernel receives the tile count as a hidden last argument.
#pragma once

#include <stdint.h>

namespace th {

constexpr uint32_t kLaunchDescMagic = 0x54484431u;  // "THD1"
constexpr uint32_t kScaleIndex = 0x3fu;    // scale_args byte: argument index + 1
constexpr uint32_t kScaleWide = 0x40u;     // ... the argument is 64-bit
constexpr uint32_t kScaleSigned = 0x80u;   // ... the argument is signed

struct LaunchDesc {
  uint32_t magic;         // kLaunchDescMagic
  uint32_t threads;       // workgroup size the kernel was built for
  uint32_t wg_per_tile;   // workgroups per logical tile (>= 1)
  uint32_t tiles_per_wg;  // logical tiles per workgroup (>= 1)
  uint32_t lds_bytes;     // dynamic LDS per workgroup
  // Work that depends on run-time scalar arguments (a loop's trip count, the
  // heads and sequence length of attention): wg_per_tile is multiplied by
  // ceil(arg[a0] / d0) and by ceil(arg[a1] / d1), where a0/a1 index the
  // kernel's integer arguments, then capped at wg_cap.  Zero fields disable a
  // factor (descriptors without them launch as before).  Each byte is
  // (a + 1) | kScaleWide | kScaleSigned: the argument is 64-bit, or a signed
  // value whose negative values count as zero.
  uint32_t scale_args;    // byte 0: a0, byte 1: a1; 0 = none
  uint32_t scale_div;     // d0 | d1 << 16 (0 reads as 1)
  uint32_t wg_cap;        // maximum workgroups per tile after scaling (0 = none)
  // Cap on the whole grid, in workgroups per compute unit (0 = none): kernels
  // that size their own work split from gridDim (the decode's KV split) are
  // launched with about as many workgroups as stay resident.
  uint32_t grid_per_cu;
};

// hardware workgroups for `tiles` logical tiles; `args` are the kernel's
// argument pointers (the driver's kernelParams convention); `cus` the device's
// compute units (for grid_per_cu)
inline uint64_t desc_grid(const LaunchDesc& d, uint64_t tiles, void* const* args = nullptr,
                          size_t nargs = 0, uint32_t cus = 0) {
  const uint64_t tpw = d.tiles_per_wg ? d.tiles_per_wg : 1;
  uint64_t wpt = d.wg_per_tile ? d.wg_per_tile : 1;
  for (int f = 0; f < 2; ++f) {
    const uint32_t b = (d.scale_args >> (8 * f)) & 0xffu;
    const uint32_t a = b & kScaleIndex;
    if (a == 0 || a > nargs || !args || !args[a - 1]) continue;
    uint64_t div = (d.scale_div >> (16 * f)) & 0xffffu;
    if (div == 0) div = 1;
    uint64_t v;
    if (b & kScaleWide) {
      const uint64_t w = *static_cast<const uint64_t*>(args[a - 1]);
      v = (b & kScaleSigned) && static_cast<int64_t>(w) < 0 ? 0 : w;
    } else {
      const uint32_t w = *static_cast<const uint32_t*>(args[a - 1]);
      v = (b & kScaleSigned) && static_cast<int32_t>(w) < 0 ? 0 : w;
    }
    if (v > 0xffffffffull) v = 0xffffffffull;   // kernels count tiles in 32 bits
    wpt *= (v + div - 1) / div;
  }
  if (d.wg_cap && wpt > d.wg_cap) wpt = d.wg_cap;
  if (wpt == 0) wpt = 1;
  uint64_t grid = (tiles + tpw - 1) / tpw * wpt;
  if (d.grid_per_cu && cus) {
    const uint64_t cap = static_cast<uint64_t>(d.grid_per_cu) * cus;
    if (grid > cap) grid = cap;
  }
  return grid;
}

}  // namespace th

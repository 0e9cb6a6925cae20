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

struct LaunchDesc {
  uint32_t magic;         // kLaunchDescMagic
  uint32_t threads;       // workgroup size the kernel was built for
  uint32_t wg_per_tile;   // workgroups per logical tile (>= 1)
  uint32_t tiles_per_wg;  // logical tiles per workgroup (>= 1)
  uint32_t lds_bytes;     // dynamic LDS per workgroup
  uint32_t reserved[3];
};

// hardware workgroups for `tiles` logical tiles
inline uint64_t desc_grid(const LaunchDesc& d, uint64_t tiles) {
  const uint64_t tpw = d.tiles_per_wg ? d.tiles_per_wg : 1;
  const uint64_t wpt = d.wg_per_tile ? d.wg_per_tile : 1;
  return (tiles + tpw - 1) / tpw * wpt;
}

}  // namespace th

// Internal helpers shared by the runtime, the tile-op entry points and the
// codegen target: thread-local error reporting mapped to the HalError
// categories of crates/tile_hal/src/error.rs:5-33.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "../../include/tilers_hip.h"

namespace th {

// Record `msg` as this thread's last error and return `code`.
int fail(int code, const std::string& msg);

// hipSuccess -> TH_OK; anything else -> `code` with "<op> failed: <name> (<n>)".
int check_hip(hipError_t err, const char* op, int code);

// Clear the last error (successful calls leave it untouched, like errno).
void clear_error();

// Make `ordinal` the current device of this thread.
int use_device(int ordinal);

// Per-device scratch used by entry points that take an optional workspace.
// Returns a device buffer of at least `bytes` on the current device (grown on
// demand, kept until process exit).
int device_scratch(size_t bytes, void** out);

// Per-(device, stream) scratch for entry points without a workspace argument:
// work queued on one stream runs in order, so calls never share the buffer
// concurrently.  At least `bytes` (grown on demand after draining that stream,
// kept until process exit).
int stream_scratch(hipStream_t stream, size_t bytes, void** out);

}  // namespace th

#define TH_TRY(expr)                 \
  do {                               \
    const int th_rc_ = (expr);       \
    if (th_rc_ != TH_OK) return th_rc_; \
  } while (0)

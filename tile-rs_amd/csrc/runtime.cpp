// HIP host runtime behind the tile_hal traits.
//
// Replaces the reference's CUDA backend (crates/tile_hal/src/cuda.rs): device
// open (cuda.rs:300-329), alloc/free (:348-361, :212-218), copies (:181-199),
// module load (:231-242) and launch (:245-288).  Differences by design:
//   - copies are asynchronous on the caller's stream (the reference ignores it);
//   - function handles are cached per name instead of looked up per launch;
//   - tile kernels emitted by the `hip` target are launched through their
//     launch descriptor (launch_desc.hpp).
#include "runtime.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "launch_desc.hpp"

namespace th {

namespace {
thread_local std::string g_last_error;

struct Scratch {
  void* ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_scratch_mu;
std::unordered_map<int, Scratch> g_scratch;
struct StreamKey {
  int dev;
  hipStream_t stream;
  bool operator==(const StreamKey& o) const { return dev == o.dev && stream == o.stream; }
};
struct StreamKeyHash {
  size_t operator()(const StreamKey& k) const {
    return std::hash<const void*>()(k.stream) ^ (static_cast<size_t>(k.dev) << 1);
  }
};
std::unordered_map<StreamKey, Scratch, StreamKeyHash> g_stream_scratch;
}  // namespace

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

void clear_error() { g_last_error.clear(); }

int check_hip(hipError_t err, const char* op, int code) {
  if (err == hipSuccess) return TH_OK;
  (void)hipGetLastError();  // clear the sticky per-thread error
  return fail(code, std::string(op) + " failed: " + hipGetErrorName(err) + " (" +
                        std::to_string(static_cast<int>(err)) + ")");
}

int use_device(int ordinal) {
  return check_hip(hipSetDevice(ordinal), "hipSetDevice", TH_DEVICE_ERROR);
}

int device_scratch(size_t bytes, void** out) {
  int dev = 0;
  TH_TRY(check_hip(hipGetDevice(&dev), "hipGetDevice", TH_DEVICE_ERROR));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  Scratch& s = g_scratch[dev];
  if (s.bytes < bytes) {
    const size_t old_bytes = s.bytes;
    if (s.ptr) {
      // a stream may still read the old buffer: drain the device first
      TH_TRY(check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize", TH_STREAM_ERROR));
      TH_TRY(check_hip(hipFree(s.ptr), "hipFree", TH_MEMORY_ERROR));
      s.ptr = nullptr;
      s.bytes = 0;
    }
    // grow geometrically so that a slowly growing request (a decode loop adding
    // one position per step) reallocates O(log n) times, not at every call
    size_t want = std::max(bytes, std::max(size_t(1) << 20, 2 * old_bytes));
    TH_TRY(check_hip(hipMalloc(&s.ptr, want), "hipMalloc", TH_MEMORY_ERROR));
    s.bytes = want;
  }
  *out = s.ptr;
  return TH_OK;
}

int stream_scratch(hipStream_t stream, size_t bytes, void** out) {
  int dev = 0;
  TH_TRY(check_hip(hipGetDevice(&dev), "hipGetDevice", TH_DEVICE_ERROR));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  Scratch& s = g_stream_scratch[StreamKey{dev, stream}];
  if (s.bytes < bytes) {
    const size_t old_bytes = s.bytes;
    if (s.ptr) {
      // earlier work on this stream may still read the old buffer
      TH_TRY(check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize", TH_STREAM_ERROR));
      TH_TRY(check_hip(hipFree(s.ptr), "hipFree", TH_MEMORY_ERROR));
      s.ptr = nullptr;
      s.bytes = 0;
    }
    size_t want = std::max(bytes, std::max(size_t(64) << 10, 2 * old_bytes));
    TH_TRY(check_hip(hipMalloc(&s.ptr, want), "hipMalloc", TH_MEMORY_ERROR));
    s.bytes = want;
  }
  *out = s.ptr;
  return TH_OK;
}

}  // namespace th

using th::check_hip;
using th::fail;

struct th_device_s {
  int ordinal = 0;
  std::string name;
  std::string arch;
  int cus = 0;
};

struct th_launcher_s {
  struct Fn {
    hipFunction_t fn = nullptr;
    bool has_desc = false;
    th::LaunchDesc desc{};
  };
  th_device dev = nullptr;
  std::vector<hipModule_t> modules;
  std::unordered_map<std::string, Fn> cache;
  std::mutex mu;
};

extern "C" {

const char* th_last_error(void) { return th::g_last_error.c_str(); }

#ifndef TH_BUILD_STAMP
#define TH_BUILD_STAMP "unstamped"
#endif
// The stamp is a hash of the sources this library was built from (written by the
// build); tests and smoke() compare it with the tree they run in.
const char* th_version(void) { return "tilers_hip 0.1.0 (gfx950) th-src:" TH_BUILD_STAMP; }

int th_backend_is_hip(const char* codegen_path) {
  return codegen_path != nullptr && std::strcmp(codegen_path, "hip") == 0;
}

int th_backend_from_env(void) {
  const char* v = std::getenv("TILERS_CODEGEN_PATH");
  if (!v) v = std::getenv("ACLRS_CODEGEN_PATH");
  // the reference defaults to "cpp" (Ascend) when neither is set
  const std::string path = v ? v : "cpp";
  if (th_backend_is_hip(path.c_str())) return TH_OK;
  return fail(TH_BACKEND_NOT_AVAILABLE, "unknown codegen path: " + path +
                                            " (this backend is selected by TILERS_CODEGEN_PATH=hip)");
}

int th_device_count(int* count) {
  if (!count) return fail(TH_RUNTIME_ERROR, "th_device_count: null output");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e == hipErrorNoDevice) {
    (void)hipGetLastError();
    n = 0;
  } else if (e != hipSuccess) {
    return check_hip(e, "hipGetDeviceCount", TH_BACKEND_NOT_AVAILABLE);
  }
  *count = n;
  return TH_OK;
}

int th_device_open(uint32_t ordinal, th_device* out) {
  if (!out) return fail(TH_DEVICE_ERROR, "th_device_open: null output");
  int n = 0;
  TH_TRY(th_device_count(&n));
  if (n == 0) return fail(TH_BACKEND_NOT_AVAILABLE, "no HIP device is visible");
  if (ordinal >= static_cast<uint32_t>(n))
    return fail(TH_DEVICE_ERROR, "device ordinal " + std::to_string(ordinal) + " out of range (" +
                                     std::to_string(n) + " devices)");
  TH_TRY(th::use_device(static_cast<int>(ordinal)));
  hipDeviceProp_t p;
  TH_TRY(check_hip(hipGetDeviceProperties(&p, static_cast<int>(ordinal)), "hipGetDeviceProperties",
                   TH_DEVICE_ERROR));
  auto* d = new th_device_s;
  d->ordinal = static_cast<int>(ordinal);
  d->name = p.name;
  d->arch = p.gcnArchName;
  if (d->name.empty()) {
    char buf[256] = {0};
    if (hipDeviceGetName(buf, sizeof(buf), static_cast<int>(ordinal)) == hipSuccess) d->name = buf;
    (void)hipGetLastError();
  }
  if (d->name.empty()) d->name = "AMD Instinct GPU (" + d->arch.substr(0, d->arch.find(':')) + ")";
  d->cus = p.multiProcessorCount;
  *out = d;
  return TH_OK;
}

int th_device_close(th_device dev) {
  delete dev;
  return TH_OK;
}

uint32_t th_device_ordinal(th_device dev) { return dev ? static_cast<uint32_t>(dev->ordinal) : 0u; }

static int copy_str(const std::string& s, char* buf, size_t len) {
  if (!buf || len == 0) return fail(TH_RUNTIME_ERROR, "null or empty output buffer");
  const size_t n = s.size() < len - 1 ? s.size() : len - 1;
  std::memcpy(buf, s.data(), n);
  buf[n] = '\0';
  return TH_OK;
}

int th_device_name(th_device dev, char* buf, size_t len) {
  if (!dev) return fail(TH_DEVICE_ERROR, "null device");
  return copy_str(dev->name, buf, len);
}

int th_device_arch(th_device dev, char* buf, size_t len) {
  if (!dev) return fail(TH_DEVICE_ERROR, "null device");
  return copy_str(dev->arch, buf, len);
}

int th_device_cu_count(th_device dev, int* cus) {
  if (!dev || !cus) return fail(TH_DEVICE_ERROR, "null device or output");
  *cus = dev->cus;
  return TH_OK;
}

int th_mem_info(th_device dev, size_t* free_bytes, size_t* total_bytes) {
  if (!dev || !free_bytes || !total_bytes) return fail(TH_DEVICE_ERROR, "null device or output");
  TH_TRY(th::use_device(dev->ordinal));
  return check_hip(hipMemGetInfo(free_bytes, total_bytes), "hipMemGetInfo", TH_DEVICE_ERROR);
}

int th_stream_create(th_device dev, th_stream* out) {
  if (!dev || !out) return fail(TH_STREAM_ERROR, "null device or output");
  TH_TRY(th::use_device(dev->ordinal));
  hipStream_t s = nullptr;
  TH_TRY(check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate",
                   TH_STREAM_ERROR));
  *out = s;
  return TH_OK;
}

int th_stream_destroy(th_stream s) {
  if (!s) return TH_OK;
  return check_hip(hipStreamDestroy(static_cast<hipStream_t>(s)), "hipStreamDestroy",
                   TH_STREAM_ERROR);
}

int th_stream_sync(th_stream s) {
  return check_hip(hipStreamSynchronize(static_cast<hipStream_t>(s)), "hipStreamSynchronize",
                   TH_STREAM_ERROR);
}

int th_malloc(th_device dev, size_t bytes, void** dptr) {
  if (!dev || !dptr) return fail(TH_MEMORY_ERROR, "null device or output");
  TH_TRY(th::use_device(dev->ordinal));
  *dptr = nullptr;
  if (bytes == 0) return TH_OK;
  return check_hip(hipMalloc(dptr, bytes), "hipMalloc", TH_MEMORY_ERROR);
}

int th_free(th_device dev, void* dptr) {
  if (!dptr) return TH_OK;
  if (dev) TH_TRY(th::use_device(dev->ordinal));
  return check_hip(hipFree(dptr), "hipFree", TH_MEMORY_ERROR);
}

int th_memcpy_htod_async(void* dst, const void* src, size_t bytes, th_stream s) {
  if (bytes == 0) return TH_OK;
  return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(s)),
                   "hipMemcpyHtoDAsync", TH_MEMORY_ERROR);
}

int th_memcpy_dtoh_async(void* dst, const void* src, size_t bytes, th_stream s) {
  if (bytes == 0) return TH_OK;
  return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, static_cast<hipStream_t>(s)),
                   "hipMemcpyDtoHAsync", TH_MEMORY_ERROR);
}

// Blocking copies (the semantics of cuMemcpyHtoD / cuMemcpyDtoH in the reference's
// CUDA HAL, crates/tile_hal/src/cuda.rs:181-199): hipMemcpy returns once the data
// has arrived.  It runs on the null stream, which does not wait for work on the
// library's (non-blocking) streams, so callers order it against such work by
// synchronizing their stream first.
int th_memcpy_htod(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return TH_OK;
  return check_hip(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpyHtoD",
                   TH_MEMORY_ERROR);
}

int th_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return TH_OK;
  return check_hip(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpyDtoH",
                   TH_MEMORY_ERROR);
}

int th_memcpy_dtod_async(void* dst, const void* src, size_t bytes, th_stream s) {
  if (bytes == 0) return TH_OK;
  return check_hip(
      hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(s)),
      "hipMemcpyDtoDAsync", TH_MEMORY_ERROR);
}

int th_memset_async(void* dst, int value, size_t bytes, th_stream s) {
  if (bytes == 0) return TH_OK;
  return check_hip(hipMemsetAsync(dst, value, bytes, static_cast<hipStream_t>(s)), "hipMemsetAsync",
                   TH_MEMORY_ERROR);
}

int th_event_create(th_event* out) {
  if (!out) return fail(TH_STREAM_ERROR, "null output");
  hipEvent_t e = nullptr;
  TH_TRY(check_hip(hipEventCreate(&e), "hipEventCreate", TH_STREAM_ERROR));
  *out = e;
  return TH_OK;
}

int th_event_destroy(th_event e) {
  if (!e) return TH_OK;
  return check_hip(hipEventDestroy(static_cast<hipEvent_t>(e)), "hipEventDestroy", TH_STREAM_ERROR);
}

int th_event_record(th_event e, th_stream s) {
  return check_hip(hipEventRecord(static_cast<hipEvent_t>(e), static_cast<hipStream_t>(s)),
                   "hipEventRecord", TH_STREAM_ERROR);
}

int th_event_sync(th_event e) {
  return check_hip(hipEventSynchronize(static_cast<hipEvent_t>(e)), "hipEventSynchronize",
                   TH_STREAM_ERROR);
}

int th_event_elapsed_ms(th_event start, th_event stop, float* ms) {
  if (!ms) return fail(TH_STREAM_ERROR, "null output");
  return check_hip(
      hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
      "hipEventElapsedTime", TH_STREAM_ERROR);
}

int th_launcher_create(th_device dev, th_launcher* out) {
  if (!dev || !out) return fail(TH_KERNEL_ERROR, "null device or output");
  auto* l = new th_launcher_s;
  l->dev = dev;
  *out = l;
  return TH_OK;
}

int th_launcher_destroy(th_launcher l) {
  if (!l) return TH_OK;
  int rc = TH_OK;
  if (th::use_device(l->dev->ordinal) == TH_OK) {
    for (hipModule_t m : l->modules) {
      const int r = check_hip(hipModuleUnload(m), "hipModuleUnload", TH_KERNEL_ERROR);
      if (rc == TH_OK) rc = r;
    }
  }
  delete l;
  return rc;
}

int th_launcher_load(th_launcher l, const char* path, th_kernel_mode mode) {
  (void)mode;  // one execution engine on CDNA4: MFMA and vector share the CU
  if (!l || !path) return fail(TH_KERNEL_ERROR, "null launcher or path");
  TH_TRY(th::use_device(l->dev->ordinal));
  hipModule_t m = nullptr;
  const hipError_t e = hipModuleLoad(&m, path);
  if (e != hipSuccess) {
    th::check_hip(e, "hipModuleLoad", TH_KERNEL_ERROR);
    return fail(TH_KERNEL_ERROR, std::string("hipModuleLoad failed for ") + path + ": " +
                                     hipGetErrorName(e) + " (" + std::to_string(int(e)) + ")");
  }
  std::lock_guard<std::mutex> lock(l->mu);
  l->modules.push_back(m);
  return TH_OK;
}

}  // extern "C"

namespace {
// The kernel `name` in the launcher's modules, with its launch descriptor (cached
// per name).
int find_kernel(th_launcher l, const char* name, th_launcher_s::Fn* out) {
  {
    std::lock_guard<std::mutex> lock(l->mu);
    auto it = l->cache.find(name);
    if (it == l->cache.end()) {
      th_launcher_s::Fn found;
      for (hipModule_t m : l->modules) {
        hipFunction_t f = nullptr;
        if (hipModuleGetFunction(&f, m, name) == hipSuccess) {
          found.fn = f;
          hipDeviceptr_t dp = nullptr;
          size_t bytes = 0;
          const std::string dname = std::string("__th_desc_") + name;
          if (hipModuleGetGlobal(&dp, &bytes, m, dname.c_str()) == hipSuccess &&
              bytes == sizeof(th::LaunchDesc)) {
            TH_TRY(check_hip(hipMemcpyDtoH(&found.desc, dp, sizeof(th::LaunchDesc)),
                             "hipMemcpyDtoH(launch descriptor)", TH_KERNEL_ERROR));
            found.has_desc = found.desc.magic == th::kLaunchDescMagic;
          }
          (void)hipGetLastError();
          break;
        }
        (void)hipGetLastError();
      }
      if (!found.fn)
        return fail(TH_KERNEL_ERROR, std::string("kernel not found in loaded modules: ") + name);
      it = l->cache.emplace(name, found).first;
    }
    *out = it->second;
  }
  return TH_OK;
}
}  // namespace

extern "C" {

int th_launcher_grid(th_launcher l, const char* name, uint32_t blocks, void** args, size_t nargs,
                     uint64_t* grid, uint32_t* threads) {
  if (!l || !name || !grid || !threads) return fail(TH_KERNEL_ERROR, "null launcher, name or output");
  TH_TRY(th::use_device(l->dev->ordinal));
  th_launcher_s::Fn fn;
  TH_TRY(find_kernel(l, name, &fn));
  if (!fn.has_desc || blocks == 0) {
    *grid = blocks;
    *threads = 0;   // the caller's block size
    return TH_OK;
  }
  *grid = th::desc_grid(fn.desc, blocks, args, nargs, static_cast<uint32_t>(l->dev->cus));
  *threads = fn.desc.threads;
  return TH_OK;
}

int th_launcher_launch(th_launcher l, const char* name, uint32_t blocks, uint32_t threads_per_block,
                       uint32_t shared_mem_bytes, void** args, size_t nargs, th_stream s) {
  if (!l || !name) return fail(TH_KERNEL_ERROR, "null launcher or kernel name");
  TH_TRY(th::use_device(l->dev->ordinal));
  th_launcher_s::Fn fn;
  TH_TRY(find_kernel(l, name, &fn));
  if (blocks == 0) return TH_OK;
  if (!fn.has_desc) {
    return check_hip(hipModuleLaunchKernel(fn.fn, blocks, 1, 1, threads_per_block, 1, 1,
                                           shared_mem_bytes, static_cast<hipStream_t>(s), args,
                                           nullptr),
                     "hipModuleLaunchKernel", TH_KERNEL_ERROR);
  }
  const uint64_t grid = th::desc_grid(fn.desc, blocks, args, nargs, static_cast<uint32_t>(l->dev->cus));
  if (grid > 0x7fffffffu) return fail(TH_KERNEL_ERROR, "launch grid too large");
  std::vector<void*> full(args, args + nargs);
  uint32_t tiles = blocks;
  full.push_back(&tiles);
  return check_hip(hipModuleLaunchKernel(fn.fn, static_cast<uint32_t>(grid), 1, 1, fn.desc.threads, 1,
                                         1, fn.desc.lds_bytes, static_cast<hipStream_t>(s),
                                         full.data(), nullptr),
                   "hipModuleLaunchKernel", TH_KERNEL_ERROR);
}

}  // extern "C"

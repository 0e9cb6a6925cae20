/*
 * tilers_hip — C ABI of the MI355X (gfx950) execution path for tile-rs's
 * tile_std matmul, row-softmax and attention tile ops.
 *
 * Three groups of entry points, each replacing one reference interface:
 *
 *   1. Host runtime (replaces tile_hal's CUDA backend, crates/tile_hal/src/cuda.rs,
 *      behind the unchanged traits Device / DeviceBuffer / Stream / KernelLauncher,
 *      crates/tile_hal/src/{device,buffer,stream,kernel}.rs).
 *   2. Tile ops (the kernels the `hip` target lowers __tile_* intrinsics to,
 *      crates/tile_std/src/tile.rs).  Device pointers in, device pointers out,
 *      enqueued on a stream.
 *   3. Codegen target (the `hip` CodegenTarget behind crates/tile_codegen/src/
 *      target.rs:57-65 and TargetRegistry, crates/tile_codegen/src/registry.rs).
 *
 * Conventions:
 *   - Every function that can fail returns an int status: TH_OK (0) or one of
 *     the six HalError categories (crates/tile_hal/src/error.rs:5-33).  The
 *     message of the last failure on the calling thread is th_last_error();
 *     driver failures read "<op> failed: <hip error name> (<code>)", the shape
 *     of check_cu in crates/tile_hal/src/cuda.rs:124-130.
 *   - No function throws across this boundary and none takes torch types.
 *   - Streams are HIP streams (hipStream_t) passed as void*; NULL means the
 *     default stream of the current device.
 *   - 16-bit floats (f16 and bf16) share the uint16_t carrier, as in tile_std
 *     (crates/tile_std/src/lib.rs:182); a th_dtype tag says which.
 */
#ifndef TILERS_HIP_H
#define TILERS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: HalError variants (crates/tile_hal/src/error.rs:5-33) ---- */
#define TH_OK 0
#define TH_DEVICE_ERROR 1          /* HalError::DeviceError */
#define TH_MEMORY_ERROR 2          /* HalError::MemoryError */
#define TH_KERNEL_ERROR 3          /* HalError::KernelError (also bad shapes/args) */
#define TH_STREAM_ERROR 4          /* HalError::StreamError */
#define TH_BACKEND_NOT_AVAILABLE 5 /* HalError::BackendNotAvailable */
#define TH_RUNTIME_ERROR 6         /* HalError::RuntimeError */

/* ---- element types: TileDtype (crates/tile_hal/src/kernel.rs:84-93) ---- */
typedef enum th_dtype { TH_F32 = 0, TH_F16 = 1, TH_BF16 = 2 } th_dtype;

/* ---- kernel modes: KernelMode (crates/tile_hal/src/kernel.rs:8-17) ---- */
typedef enum th_kernel_mode { TH_MODE_VECTOR = 0, TH_MODE_MATRIX = 1, TH_MODE_GENERAL = 2 } th_kernel_mode;

typedef struct th_device_s* th_device;
typedef struct th_launcher_s* th_launcher;
typedef void* th_stream;

/* Message of the last failed call on this thread ("" when none). */
const char* th_last_error(void);
/* Library version string. */
const char* th_version(void);

/* ======================================================================== */
/* 1. Host runtime                                                           */
/* ======================================================================== */

/* Backend selection: BackendKind::from_codegen_path / BackendSelector::from_env
 * (crates/tile_hal/src/backend.rs:27-40, :70-78).  Returns 1 when `name` selects
 * this backend ("hip"), 0 otherwise.  th_backend_from_env reads
 * TILERS_CODEGEN_PATH, then ACLRS_CODEGEN_PATH; TH_OK when it names "hip",
 * TH_BACKEND_NOT_AVAILABLE otherwise (the message names the value). */
int th_backend_is_hip(const char* codegen_path);
int th_backend_from_env(void);

/* Number of visible HIP devices (0 when no GPU or no driver). */
int th_device_count(int* count);

/* Device (crates/tile_hal/src/device.rs:25-57; CudaDevice::new cuda.rs:300-329). */
int th_device_open(uint32_t ordinal, th_device* out);
int th_device_close(th_device dev);
uint32_t th_device_ordinal(th_device dev);
/* Copies the device name (e.g. "AMD Instinct MI355X") into buf (NUL-terminated). */
int th_device_name(th_device dev, char* buf, size_t len);
/* gfx architecture name, e.g. "gfx950". */
int th_device_arch(th_device dev, char* buf, size_t len);
int th_mem_info(th_device dev, size_t* free_bytes, size_t* total_bytes);
/* Number of compute units. */
int th_device_cu_count(th_device dev, int* cus);

/* Streams (crates/tile_hal/src/stream.rs:7-10).  Default priority only. */
int th_stream_create(th_device dev, th_stream* out);
int th_stream_destroy(th_stream s);
int th_stream_sync(th_stream s);

/* Buffers (crates/tile_hal/src/buffer.rs:32-54; Device::alloc device.rs:44).
 * Copies are asynchronous on the given stream (unlike cuda.rs:181-199, which
 * ignores it); host memory must stay valid until the stream is synchronized. */
int th_malloc(th_device dev, size_t bytes, void** dptr);
int th_free(th_device dev, void* dptr);
int th_memcpy_htod_async(void* dst, const void* src, size_t bytes, th_stream s);
int th_memcpy_dtoh_async(void* dst, const void* src, size_t bytes, th_stream s);
/* Blocking copies with the semantics of the reference CUDA HAL's
 * cuMemcpyHtoD / cuMemcpyDtoH (crates/tile_hal/src/cuda.rs:181-199): they return
 * once the data has arrived.  They run on the null stream, which does not wait
 * for work on streams from th_stream_create (non-blocking): synchronize such a
 * stream first when it may still write (or read) the device buffer. */
int th_memcpy_htod(void* dst, const void* src, size_t bytes);
int th_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int th_memcpy_dtod_async(void* dst, const void* src, size_t bytes, th_stream s);
int th_memset_async(void* dst, int value, size_t bytes, th_stream s);

/* Events (timing; no reference counterpart — the reference has no timing API). */
typedef void* th_event;
int th_event_create(th_event* out);
int th_event_destroy(th_event e);
int th_event_record(th_event e, th_stream s);
int th_event_sync(th_event e);
int th_event_elapsed_ms(th_event start, th_event stop, float* ms);

/* Kernel launcher (crates/tile_hal/src/kernel.rs:23-42; cuda.rs:231-288).
 * load: hipModuleLoad of a code object (.hsaco).  launch: by kernel name with a
 * 1-D LaunchGrid and `args` = array of pointers TO argument values (the
 * kernelParams convention of the reference).  Function handles are cached per
 * name (the reference looks them up on every launch, cuda.rs:252-262).
 *
 * Kernels emitted by the `hip` target carry a launch descriptor
 * (`__th_desc_<name>`, see tile-rs_amd/csrc/target/launch_desc.hpp): `blocks`
 * is then the number of logical tiles (the #[tile_kernel] grid, crates/
 * tile_std_macros/src/lib.rs:217-266) and the launcher expands it to the
 * hardware grid and block size the kernel was built for, appending the tile
 * count as a hidden trailing argument.  Kernels without a descriptor launch
 * exactly as given. */
int th_launcher_create(th_device dev, th_launcher* out);
int th_launcher_destroy(th_launcher l);
int th_launcher_load(th_launcher l, const char* path, th_kernel_mode mode);
int th_launcher_launch(th_launcher l, const char* name, uint32_t blocks, uint32_t threads_per_block,
                       uint32_t shared_mem_bytes, void** args, size_t nargs, th_stream s);
/* The hardware grid (workgroups) and workgroup size th_launcher_launch would use
 * for the same arguments, without launching; `*threads` = 0 for a kernel without
 * a descriptor (it runs with the caller's block size).  No reference
 * counterpart: the reference launches exactly the grid it is given. */
int th_launcher_grid(th_launcher l, const char* name, uint32_t blocks, void** args, size_t nargs,
                     uint64_t* grid, uint32_t* threads);

/* ======================================================================== */
/* 2. Tile ops                                                                */
/* ======================================================================== */

/* Row softmax over `cols` for `rows` rows, row-major.  x and y may alias.
 * __tile_softmax_f32 (tile.rs:190, :2297) for TH_F32; __tile_softmax_f16
 * (tile.rs:2163, :2912) for TH_F16, and TH_BF16 on the same u16 carrier.
 * Semantics: linalg.softmax dimension(1) (mlir_to_linalg.rs:1305-1343). */
int th_softmax(const void* x, void* y, uint32_t rows, uint32_t cols, th_dtype dtype, th_stream s);

/* C = A * B with f32 accumulation (linalg.fill 0 + linalg.matmul,
 * mlir_to_linalg.rs:1345-1393).  A is M x K; B is K x N, or N x K when
 * b_transposed != 0.  in_dtype applies to A and B; out_dtype to C.
 *   __tile_matmul_f32           tile.rs:193, :2309   in=F32  out=F32
 *   __tile_matmul_f16           tile.rs:1983, :2593  in=F16/BF16  out=F16/BF16
 *   tile_matmul_f16_acc_f32     tile.rs:2666         in=F16/BF16  out=F32
 *   __tile_matmul_transposed_*  tile.rs:2022, :2028, :2694   b_transposed=1
 * `batch` stacked problems with element strides sa, sb, sc (0 = dense). */
int th_matmul(const void* a, const void* b, void* c, uint32_t m, uint32_t k, uint32_t n,
              th_dtype in_dtype, th_dtype out_dtype, int b_transposed, uint32_t batch,
              uint64_t sa, uint64_t sb, uint64_t sc, th_stream s);

/* GEMM with the SiLU*Mul epilogue fused: C = silu(A.B) * UP, elementwise, where
 * silu(x) = x / (1 + exp(-x)).  Replaces the tile chain matmul -> __tile_silu_*
 * -> __tile_mul_* (tile.rs:229, :1135; linalg mlir_to_linalg.rs:449-451,
 * :774-782, :425; the gpu target fuses silu+mul the same way,
 * mlir_to_gpu.rs:536-634).  UP has out_dtype and C's layout and strides;
 * arithmetic is f32 with one rounding at the output (whole 256 x 256 tiles with
 * 16-bit C evaluate exp and the division with the hardware's f32 exp2 and
 * reciprocal, within the GEMM tolerance of the exact form).  Other arguments as
 * th_matmul. */
int th_matmul_silu_mul(const void* a, const void* b, const void* up, void* c, uint32_t m,
                       uint32_t k, uint32_t n, th_dtype in_dtype, th_dtype out_dtype,
                       int b_transposed, uint32_t batch, uint64_t sa, uint64_t sb, uint64_t sc,
                       th_stream s);

/* Row RMSNorm (__tile_rms_norm_f32(dst, src, eps, rows, cols), tile.rs:2063;
 * linalg mlir_to_linalg.rs:1666-1763): y = x * rsqrt(sum(x^2) / cols + eps) per
 * row, f32 math for every dtype.  eps must be >= 0. */
int th_rms_norm(const void* x, void* y, uint32_t rows, uint32_t cols, float eps, th_dtype dtype,
                th_stream s);

/* Causal mask (__tile_causal_mask_f32, tile.rs:1877, :2435; linalg
 * mlir_to_linalg.rs:1191-1247): y[r][c] = x[r][c] if c <= r else -inf, for
 * `tiles` stacked rows x cols tiles. */
int th_causal_mask_f32(const float* x, float* y, uint32_t rows, uint32_t cols, uint32_t tiles,
                       th_stream s);

/* Single-head, non-causal attention softmax(Q K^T / sqrt(D)) V on S x D tiles
 * (__tile_attention_f32, tile.rs:221, :2401; linalg mlir_to_linalg.rs:1781-1902).
 * `tiles` stacked problems. */
int th_attention(const void* q, const void* k, const void* v, void* o, uint32_t seq_len,
                 uint32_t head_dim, uint32_t tiles, th_dtype dtype, th_stream s);

/* Causal GQA prefill (__tile_attention_prefill_f32, tile.rs:2136, :3064;
 * runtime params mlir_to_msl.rs:1851-1859 in the same order).
 * Q, O: [batch][seq_len][num_heads][head_dim]; K, V: [batch][num_kv_heads][max_seq][head_dim].
 * Query qi sees KV positions <= start_pos + qi (start_pos + seq_len <= max_seq). */
int th_attention_prefill(const void* q, const void* k, const void* v, void* o, uint32_t batch,
                         uint32_t seq_len, uint32_t start_pos, uint32_t max_seq,
                         uint32_t head_dim, uint32_t num_heads, uint32_t num_kv_heads,
                         th_dtype dtype, th_stream s);

/* GQA decode, one query token (__tile_attention_decode_f32, tile.rs:2124, :3011;
 * runtime params mlir_to_msl.rs:1816-1823 in the same order).
 * Q, O: [batch][num_heads][head_dim]; K, V: [batch][num_kv_heads][max_seq][head_dim];
 * positions [0, seq_len) are attended.
 * `workspace` may be NULL (the library keeps one per device, grown on demand;
 * calls that overlap on one device then race on it) or a device buffer of at
 * least th_attention_decode_workspace_size(...) bytes (non-zero for head_dim 128
 * and for head dims below 128 that are multiples of 8: 64 runs natively, the others
 * run padded to 128; the size covers 128-column records either way). */
size_t th_attention_decode_workspace_size(uint32_t batch, uint32_t seq_len, uint32_t head_dim,
                                          uint32_t num_heads, uint32_t num_kv_heads);
int th_attention_decode(const void* q, const void* k, const void* v, void* o, uint32_t batch,
                        uint32_t seq_len, uint32_t max_seq, uint32_t head_dim,
                        uint32_t num_heads, uint32_t num_kv_heads, th_dtype dtype,
                        void* workspace, size_t workspace_bytes, th_stream s);

/* th_attention_decode that allocates nothing.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same result
 * as th_attention_decode.  The split partials go to a fixed 8 MiB array in each
 * GPU's memory that is loaded with the library's code object and held until the
 * process ends; a plan whose partials would need more returns TH_MEMORY_ERROR,
 * and head dims below 128 other than 64 (which run on padded copies) return
 * TH_KERNEL_ERROR.
 * Every call on one GPU shares that GPU's array, so calls that overlap on one
 * GPU (on different streams, or replays of captured graphs running at the same
 * time) race on it; calls ordered on one stream do not. */
int th_attention_decode_static(const void* q, const void* k, const void* v, void* o,
                               uint32_t batch, uint32_t seq_len, uint32_t max_seq,
                               uint32_t head_dim, uint32_t num_heads, uint32_t num_kv_heads,
                               th_dtype dtype, th_stream s);

/* Synthetic data: fill `n` elements with i.i.d. samples, counter-based and
 * seeded (element i depends only on (seed, i)).  dist 0 = Uniform[p0, p1),
 * dist 1 = Normal(mean p0, std p1).  For benchmarks and tests only; no
 * reference counterpart. */
int th_fill_random(void* dst, uint64_t n, th_dtype dtype, int dist, float p0, float p1,
                   uint64_t seed, th_stream s);

/* ======================================================================== */
/* 3. Codegen target and registry                                             */
/* ======================================================================== */

/* EmitOpts / HardwareParams (crates/tile_codegen/src/target.rs:17-26). */
typedef struct th_emit_opts {
  size_t ub_size; /* ignored by the hip target */
} th_emit_opts;

/* The hip target's name(): "hip" (target.rs:60-62). */
const char* th_target_name(void);

/* CodegenTarget::emit (target.rs:64): pure and deterministic MLIR text -> HIP
 * source.  On success *out_src (HIP C++), *out_ext ("hip") and *out_meta (JSON
 * TargetMeta: {"has_cube_kernel":false,"kernel_names":[...]}) are set and the
 * caller frees out_src / out_meta with th_string_free.  On failure returns
 * TH_KERNEL_ERROR and *out_err holds the message (free with th_string_free). */
int th_emit(const char* mlir, size_t len, const th_emit_opts* opts, char** out_src,
            const char** out_ext, char** out_meta, char** out_err);
void th_string_free(char* s);

/* Host-side toolchain step that the reference keeps outside the trait
 * (target.rs:1-9): compile emitted source to a gfx950 code object with hipcc.
 * `include_dir` may be NULL (the library's own kernel headers are used). */
int th_compile(const char* src, size_t len, const char* out_path, const char* include_dir,
               char** out_err);

/* TargetRegistry (crates/tile_codegen/src/registry.rs:19-68) with the built-in
 * targets of this library: "debug" (DebugTarget, targets.rs:32-53) and "hip".
 * select() returns the first registered target of that name. */
typedef struct th_registry_s* th_registry;
typedef int (*th_emit_fn)(const char* mlir, size_t len, const th_emit_opts* opts, char** out_src,
                          const char** out_ext, char** out_meta, char** out_err);
th_registry th_registry_new(void);
th_registry th_registry_with_builtin(void);
void th_registry_free(th_registry r);
/* register(): `name` and `ext` are copied.  EmitterTarget::new(name, ext, f)
 * (targets.rs:82-101) is this call with a plain emit function. */
int th_registry_register(th_registry r, const char* name, const char* ext, th_emit_fn emit);
size_t th_registry_len(th_registry r);
/* names(): writes up to `cap` borrowed name pointers; returns the count. */
size_t th_registry_names(th_registry r, const char** names, size_t cap);
/* select(name) + emit: TH_BACKEND_NOT_AVAILABLE when no target has that name
 * (message lists the available ones). */
int th_registry_emit(th_registry r, const char* name, const char* mlir, size_t len,
                     const th_emit_opts* opts, char** out_src, const char** out_ext,
                     char** out_meta, char** out_err);

#ifdef __cplusplus
}
#endif

#endif /* TILERS_HIP_H */

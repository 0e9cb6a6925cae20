"""tilers_hip — host-side mirror of tile-rs's tile_hal and tile_codegen interfaces
over the MI355X C ABI (include/tilers_hip.h, libtilers_hip.so).

Names and argument meaning follow the reference's Rust API:
  Device            crates/tile_hal/src/device.rs:25-57     -> HipDevice
  DeviceBuffer<T>   crates/tile_hal/src/buffer.rs:32-54     -> HipBuffer
  Stream            crates/tile_hal/src/stream.rs:7-10      -> HipStream
  KernelLauncher    crates/tile_hal/src/kernel.rs:23-42     -> HipLauncher
  LaunchGrid        crates/tile_hal/src/kernel.rs:46-79     -> LaunchGrid
  KernelMode        crates/tile_hal/src/kernel.rs:8-17      -> KernelMode
  TileDtype         crates/tile_hal/src/kernel.rs:84-93     -> TileDtype
  HalError          crates/tile_hal/src/error.rs:5-35       -> HalError
  BackendSelector   crates/tile_hal/src/backend.rs:63-112   -> BackendSelector
  CodegenTarget     crates/tile_codegen/src/target.rs:57-65 -> CodegenTarget
  TargetRegistry    crates/tile_codegen/src/registry.rs     -> TargetRegistry
  EmitterTarget     crates/tile_codegen/src/targets.rs:82-101 -> EmitterTarget
The tile ops (section 2 of the header) are plain functions taking device
buffers or raw device pointers.  Everything runs through the HIP library; a
missing library is an error, never a fallback.
"""
from __future__ import annotations

import ctypes as C
import enum
import os
from dataclasses import dataclass, field
from typing import Callable, Optional, Sequence

import numpy as np

from ._lib import (EMIT_FN, TH_BACKEND_NOT_AVAILABLE, TH_KERNEL_ERROR, TH_OK, EmitOpts, HalError,
                   check, load)

__all__ = [
    "HalError", "TileDtype", "KernelMode", "LaunchGrid", "MemInfo", "HipDevice", "HipStream",
    "HipBuffer", "HipLauncher", "HipEvent", "BackendSelector", "BackendKind", "EmitOut",
    "TargetMeta", "CodegenTarget", "EmitterTarget", "TargetRegistry", "softmax", "matmul",
    "matmul_silu_mul", "rms_norm", "causal_mask_f32", "attention", "attention_prefill", "attention_decode",
    "attention_decode_workspace_size", "fill_random", "compile_source", "device_count", "lib",
]


def lib():
    return load()


class TileDtype(enum.IntEnum):
    """TileDtype subset the hot path uses (crates/tile_hal/src/kernel.rs:84-93)."""
    F32 = 0
    F16 = 1
    BF16 = 2

    @property
    def itemsize(self) -> int:
        return 4 if self == TileDtype.F32 else 2

    @property
    def host_dtype(self):
        return np.float32 if self == TileDtype.F32 else np.uint16


class KernelMode(enum.IntEnum):
    VECTOR = 0
    MATRIX = 1
    GENERAL = 2


@dataclass
class LaunchGrid:
    """1-D launch dimensions (crates/tile_hal/src/kernel.rs:46-79)."""
    blocks: int
    threads_per_block: int = 1
    shared_mem_bytes: int = 0

    @staticmethod
    def blocks_only(n: int) -> "LaunchGrid":  # LaunchGrid::blocks
        return LaunchGrid(n, 1, 0)

    @staticmethod
    def cuda(blocks: int, threads: int) -> "LaunchGrid":  # LaunchGrid::cuda
        return LaunchGrid(blocks, threads, 0)

    def with_shared_mem(self, nbytes: int) -> "LaunchGrid":
        self.shared_mem_bytes = nbytes
        return self


@dataclass
class MemInfo:
    free: int
    total: int

    def used(self) -> int:
        return self.total - self.free


def device_count() -> int:
    n = C.c_int(0)
    check(lib().th_device_count(C.byref(n)))
    return n.value


class HipStream:
    """Stream (crates/tile_hal/src/stream.rs:7-10); destroyed on close/GC."""

    def __init__(self, handle: int | None):
        self.handle = handle

    def synchronize(self) -> None:
        check(lib().th_stream_sync(self.handle))

    def close(self) -> None:
        if self.handle:
            check(lib().th_stream_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            if self.handle:
                lib().th_stream_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class HipEvent:
    def __init__(self):
        h = C.c_void_p()
        check(lib().th_event_create(C.byref(h)))
        self.handle = h.value

    def record(self, stream: HipStream) -> None:
        check(lib().th_event_record(self.handle, stream.handle))

    def synchronize(self) -> None:
        check(lib().th_event_sync(self.handle))

    def elapsed_ms(self, end: "HipEvent") -> float:
        ms = C.c_float(0.0)
        check(lib().th_event_elapsed_ms(self.handle, end.handle, C.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                lib().th_event_destroy(self.handle)
        except Exception:
            pass


class HipBuffer:
    """Owned device allocation of `count` elements (crates/tile_hal/src/buffer.rs:32-54)."""

    def __init__(self, device: "HipDevice", count: int, dtype: TileDtype):
        self.device = device
        self.count = int(count)
        self.dtype = TileDtype(dtype)
        self.nbytes = self.count * self.dtype.itemsize
        p = C.c_void_p()
        check(lib().th_malloc(device.handle, self.nbytes, C.byref(p)))
        self.ptr = p.value or 0

    def __len__(self) -> int:
        return self.count

    def is_empty(self) -> bool:
        return self.count == 0

    def copy_from_host(self, src: np.ndarray, stream: HipStream) -> None:
        arr = np.ascontiguousarray(src)
        if arr.nbytes != self.nbytes:
            raise HalError(2, f"copy_from_host: {arr.nbytes} bytes into a {self.nbytes}-byte buffer")
        self._pin = arr  # must outlive the asynchronous copy
        check(lib().th_memcpy_htod_async(self.ptr, arr.ctypes.data, self.nbytes, stream.handle))

    def copy_to_host(self, stream: HipStream) -> np.ndarray:
        out = np.empty(self.count, dtype=self.dtype.host_dtype)
        check(lib().th_memcpy_dtoh_async(out.ctypes.data, self.ptr, self.nbytes, stream.handle))
        stream.synchronize()
        return out

    def as_raw_ptr(self) -> int:
        return self.ptr

    def as_raw_mut_ptr(self) -> int:
        return self.ptr

    def free(self) -> None:
        if self.ptr:
            check(lib().th_free(self.device.handle, self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            if self.ptr:
                lib().th_free(self.device.handle, self.ptr)
                self.ptr = 0
        except Exception:
            pass


class HipLauncher:
    """KernelLauncher over hipModuleLoad / hipModuleLaunchKernel (kernel.rs:23-42)."""

    def __init__(self, device: "HipDevice"):
        h = C.c_void_p()
        check(lib().th_launcher_create(device.handle, C.byref(h)))
        self.handle = h.value
        self.device = device

    def load(self, path: str | os.PathLike, mode: KernelMode = KernelMode.VECTOR) -> None:
        check(lib().th_launcher_load(self.handle, os.fspath(path).encode(), int(mode)))

    @staticmethod
    def _params(args):
        holders = list(args)
        arr = (C.c_void_p * max(1, len(holders)))()
        for i, a in enumerate(holders):
            arr[i] = C.cast(C.pointer(a), C.c_void_p)
        return holders, arr

    def launch(self, name: str, grid: LaunchGrid, args: Sequence[C._SimpleCData | C.c_void_p],
               stream: HipStream) -> None:
        """`args` are ctypes values; pointers to them form the kernelParams array."""
        holders, arr = self._params(args)
        check(lib().th_launcher_launch(self.handle, name.encode(), grid.blocks,
                                       grid.threads_per_block, grid.shared_mem_bytes, arr,
                                       len(holders), stream.handle))

    def hardware_grid(self, name: str, grid: LaunchGrid,
                      args: Sequence[C._SimpleCData | C.c_void_p]) -> tuple[int, int]:
        """(workgroups, threads per workgroup) that `launch` would use; threads is 0
        for a kernel without a launch descriptor."""
        holders, arr = self._params(args)
        g, t = C.c_uint64(), C.c_uint32()
        check(lib().th_launcher_grid(self.handle, name.encode(), grid.blocks, arr, len(holders),
                                     C.byref(g), C.byref(t)))
        return g.value, t.value

    def __del__(self):
        try:
            if self.handle:
                lib().th_launcher_destroy(self.handle)
        except Exception:
            pass


class HipDevice:
    """Device (crates/tile_hal/src/device.rs:25-57) on one MI355X."""

    def __init__(self, ordinal: int = 0):
        h = C.c_void_p()
        check(lib().th_device_open(int(ordinal), C.byref(h)))
        self.handle = h.value

    @staticmethod
    def new(ordinal: int = 0) -> "HipDevice":
        return HipDevice(ordinal)

    def ordinal(self) -> int:
        return lib().th_device_ordinal(self.handle)

    def name(self) -> str:
        buf = C.create_string_buffer(256)
        check(lib().th_device_name(self.handle, buf, 256))
        return buf.value.decode()

    def arch(self) -> str:
        buf = C.create_string_buffer(64)
        check(lib().th_device_arch(self.handle, buf, 64))
        return buf.value.decode()

    def cu_count(self) -> int:
        n = C.c_int(0)
        check(lib().th_device_cu_count(self.handle, C.byref(n)))
        return n.value

    def create_stream(self) -> HipStream:
        h = C.c_void_p()
        check(lib().th_stream_create(self.handle, C.byref(h)))
        return HipStream(h.value)

    def alloc(self, count: int, dtype: TileDtype = TileDtype.F32) -> HipBuffer:
        return HipBuffer(self, count, dtype)

    def alloc_from_slice(self, data: np.ndarray, stream: HipStream,
                         dtype: Optional[TileDtype] = None) -> HipBuffer:
        if dtype is None:
            dtype = TileDtype.F32 if data.dtype == np.float32 else TileDtype.BF16
        buf = HipBuffer(self, data.size, dtype)
        buf.copy_from_host(data, stream)
        return buf

    def mem_info(self) -> MemInfo:
        f, t = C.c_size_t(0), C.c_size_t(0)
        check(lib().th_mem_info(self.handle, C.byref(f), C.byref(t)))
        return MemInfo(f.value, t.value)

    def create_launcher(self) -> HipLauncher:
        return HipLauncher(self)

    def close(self) -> None:
        if self.handle:
            lib().th_device_close(self.handle)
            self.handle = None


class BackendKind(enum.Enum):
    Hip = "hip"


class BackendSelector:
    """BackendSelector (crates/tile_hal/src/backend.rs:63-112) for the hip backend."""

    def __init__(self, kind: BackendKind = BackendKind.Hip):
        self._kind = kind

    @staticmethod
    def from_codegen_path(s: str) -> Optional[BackendKind]:
        return BackendKind.Hip if lib().th_backend_is_hip(s.encode()) else None

    @staticmethod
    def from_env() -> "BackendSelector":
        check(lib().th_backend_from_env())
        return BackendSelector(BackendKind.Hip)

    def kind(self) -> BackendKind:
        return self._kind

    def device(self, ordinal: int = 0) -> HipDevice:
        return HipDevice(ordinal)


# ---- tile ops ----------------------------------------------------------------------

def _p(x) -> int:
    return x.as_raw_ptr() if isinstance(x, HipBuffer) else int(x or 0)


def _s(stream: Optional[HipStream]):
    return stream.handle if stream is not None else None


def softmax(x, y, rows: int, cols: int, dtype: TileDtype = TileDtype.F32,
            stream: Optional[HipStream] = None) -> None:
    check(lib().th_softmax(_p(x), _p(y), rows, cols, int(dtype), _s(stream)))


def matmul(a, b, c, m: int, k: int, n: int, in_dtype: TileDtype, out_dtype: TileDtype,
           b_transposed: bool = False, batch: int = 1, sa: int = 0, sb: int = 0, sc: int = 0,
           stream: Optional[HipStream] = None) -> None:
    check(lib().th_matmul(_p(a), _p(b), _p(c), m, k, n, int(in_dtype), int(out_dtype),
                          int(bool(b_transposed)), batch, sa, sb, sc, _s(stream)))


def matmul_silu_mul(a, b, up, c, m: int, k: int, n: int, in_dtype: TileDtype,
                    out_dtype: TileDtype, b_transposed: bool = False, batch: int = 1, sa: int = 0,
                    sb: int = 0, sc: int = 0, stream: Optional[HipStream] = None) -> None:
    """C = silu(A.B) * UP (the matmul -> silu -> mul tile chain in one kernel)."""
    check(lib().th_matmul_silu_mul(_p(a), _p(b), _p(up), _p(c), m, k, n, int(in_dtype),
                                   int(out_dtype), int(bool(b_transposed)), batch, sa, sb, sc,
                                   _s(stream)))


def rms_norm(x, y, rows: int, cols: int, eps: float, dtype: TileDtype = TileDtype.F32,
             stream: Optional[HipStream] = None) -> None:
    """y = x * rsqrt(mean(x^2, row) + eps) per row (__tile_rms_norm_f32)."""
    check(lib().th_rms_norm(_p(x), _p(y), rows, cols, float(eps), int(dtype), _s(stream)))


def causal_mask_f32(x, y, rows: int, cols: int, tiles: int = 1,
                    stream: Optional[HipStream] = None) -> None:
    check(lib().th_causal_mask_f32(_p(x), _p(y), rows, cols, tiles, _s(stream)))


def attention(q, k, v, o, seq_len: int, head_dim: int, tiles: int = 1,
              dtype: TileDtype = TileDtype.F32, stream: Optional[HipStream] = None) -> None:
    check(lib().th_attention(_p(q), _p(k), _p(v), _p(o), seq_len, head_dim, tiles, int(dtype),
                             _s(stream)))


def attention_prefill(q, k, v, o, batch: int, seq_len: int, start_pos: int, max_seq: int,
                      head_dim: int, num_heads: int, num_kv_heads: int,
                      dtype: TileDtype = TileDtype.BF16,
                      stream: Optional[HipStream] = None) -> None:
    check(lib().th_attention_prefill(_p(q), _p(k), _p(v), _p(o), batch, seq_len, start_pos,
                                     max_seq, head_dim, num_heads, num_kv_heads, int(dtype),
                                     _s(stream)))


def attention_decode_workspace_size(batch: int, seq_len: int, head_dim: int, num_heads: int,
                                    num_kv_heads: int) -> int:
    return lib().th_attention_decode_workspace_size(batch, seq_len, head_dim, num_heads,
                                                    num_kv_heads)


def attention_decode(q, k, v, o, batch: int, seq_len: int, max_seq: int, head_dim: int,
                     num_heads: int, num_kv_heads: int, dtype: TileDtype = TileDtype.BF16,
                     workspace=None, workspace_bytes: int = 0,
                     stream: Optional[HipStream] = None) -> None:
    check(lib().th_attention_decode(_p(q), _p(k), _p(v), _p(o), batch, seq_len, max_seq, head_dim,
                                    num_heads, num_kv_heads, int(dtype), _p(workspace),
                                    workspace_bytes, _s(stream)))


def fill_random(dst, n: int, dtype: TileDtype, dist: str, p0: float, p1: float, seed: int,
                stream: Optional[HipStream] = None) -> None:
    d = {"uniform": 0, "normal": 1}[dist]
    check(lib().th_fill_random(_p(dst), n, int(dtype), d, p0, p1, seed, _s(stream)))


# ---- codegen target / registry --------------------------------------------------------

@dataclass
class TargetMeta:
    has_cube_kernel: bool = False
    kernel_names: list = field(default_factory=list)


@dataclass
class EmitOut:
    source: str
    ext: str
    meta: TargetMeta


def _take_str(p: C.c_char_p) -> str:
    if not p:
        return ""
    s = C.cast(p, C.c_char_p).value.decode()
    lib().th_string_free(C.cast(p, C.c_void_p))
    return s


def _emit_call(fn, *prefix, mlir: str, ub_size: int = 0) -> EmitOut:
    import json
    data = mlir.encode()
    opts = EmitOpts(ub_size)
    src, ext, meta, err = C.c_char_p(), C.c_char_p(), C.c_char_p(), C.c_char_p()
    rc = fn(*prefix, data, len(data), C.byref(opts), C.byref(src), C.byref(ext), C.byref(meta),
            C.byref(err))
    if rc != TH_OK:
        msg = _take_str(err) or lib().th_last_error().decode()
        raise HalError(rc, msg)
    m = json.loads(_take_str(meta) or "{}")
    return EmitOut(_take_str(src), ext.value.decode() if ext.value else "",
                   TargetMeta(bool(m.get("has_cube_kernel", False)),
                              list(m.get("kernel_names", []))))


class CodegenTarget:
    """A target selected from a registry (crates/tile_codegen/src/target.rs:57-65)."""

    def __init__(self, registry: "TargetRegistry", name: str):
        self._registry = registry
        self._name = name

    def name(self) -> str:
        return self._name

    def emit(self, mlir_text: str, ub_size: int = 0) -> EmitOut:
        return _emit_call(lib().th_registry_emit, self._registry.handle, self._name.encode(),
                          mlir=mlir_text, ub_size=ub_size)


class EmitterTarget:
    """EmitterTarget::new(name, ext, f) (crates/tile_codegen/src/targets.rs:82-101):
    lifts a plain `f(mlir) -> str` (raising ValueError for Err) into a target."""

    def __init__(self, name: str, ext: str, f: Callable[[str], str]):
        self.name = name
        self.ext = ext
        self.f = f
        self._cb = None

    def _callback(self):
        if self._cb is None:
            def cb(mlir, n, _opts, out_src, out_ext, out_meta, out_err):
                text = C.string_at(mlir, n).decode()
                try:
                    src = self.f(text)
                except Exception as e:  # Err(String)
                    out_err[0] = _dup(str(e))
                    return TH_KERNEL_ERROR
                out_src[0] = _dup(src)
                out_ext[0] = C.cast(self._ext_buf, C.c_char_p)
                out_meta[0] = _dup('{"has_cube_kernel":false,"kernel_names":[]}')
                return TH_OK
            self._ext_buf = C.create_string_buffer(self.ext.encode())
            self._cb = EMIT_FN(cb)
        return self._cb


_libc = C.CDLL(None)
_libc.malloc.restype = C.c_void_p
_libc.malloc.argtypes = [C.c_size_t]


def _dup(s: str) -> C.c_char_p:
    """malloc'd copy (freed by th_string_free on the library side)."""
    b = s.encode()
    p = _libc.malloc(len(b) + 1)
    C.memmove(p, b, len(b))
    C.memset(p + len(b), 0, 1)
    return C.cast(p, C.c_char_p)


class TargetRegistry:
    """TargetRegistry (crates/tile_codegen/src/registry.rs:19-68)."""

    def __init__(self, handle=None):
        self.handle = handle if handle is not None else lib().th_registry_new()
        self._keep = []

    @staticmethod
    def new() -> "TargetRegistry":
        return TargetRegistry()

    @staticmethod
    def with_builtin() -> "TargetRegistry":
        return TargetRegistry(lib().th_registry_with_builtin())

    def register(self, target: EmitterTarget) -> None:
        cb = target._callback()
        self._keep.append(target)
        check(lib().th_registry_register(self.handle, target.name.encode(), target.ext.encode(), cb))

    def select(self, name: str) -> Optional[CodegenTarget]:
        return CodegenTarget(self, name) if name in self.names() else None

    def names(self) -> list:
        n = lib().th_registry_len(self.handle)
        arr = (C.c_char_p * max(1, n))()
        got = lib().th_registry_names(self.handle, arr, n)
        return [arr[i].decode() for i in range(got)]

    def __len__(self) -> int:
        return lib().th_registry_len(self.handle)

    def is_empty(self) -> bool:
        return len(self) == 0

    def __del__(self):
        try:
            if self.handle:
                lib().th_registry_free(self.handle)
                self.handle = None
        except Exception:
            pass


def target_name() -> str:
    return lib().th_target_name().decode()


def emit(mlir_text: str, ub_size: int = 0) -> EmitOut:
    """The hip target's emit() (th_emit)."""
    return _emit_call(lib().th_emit, mlir=mlir_text, ub_size=ub_size)


def compile_source(source: str, out_path: str | os.PathLike, include_dir: str | None = None) -> None:
    """hipcc the emitted source into a gfx950 code object (th_compile)."""
    data = source.encode()
    err = C.c_char_p()
    rc = lib().th_compile(data, len(data), os.fspath(out_path).encode(),
                          include_dir.encode() if include_dir else None, C.byref(err))
    if rc != TH_OK:
        raise HalError(rc, _take_str(err) or lib().th_last_error().decode())

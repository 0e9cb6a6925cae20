"""ctypes declarations of libtilers_hip.so (include/tilers_hip.h).

Loading fails loudly: there is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

from ._build import library_path

# status codes (include/tilers_hip.h; HalError variants, crates/tile_hal/src/error.rs:5-33)
TH_OK = 0
TH_DEVICE_ERROR = 1
TH_MEMORY_ERROR = 2
TH_KERNEL_ERROR = 3
TH_STREAM_ERROR = 4
TH_BACKEND_NOT_AVAILABLE = 5
TH_RUNTIME_ERROR = 6

ERROR_KINDS = {
    TH_DEVICE_ERROR: "DeviceError",
    TH_MEMORY_ERROR: "MemoryError",
    TH_KERNEL_ERROR: "KernelError",
    TH_STREAM_ERROR: "StreamError",
    TH_BACKEND_NOT_AVAILABLE: "BackendNotAvailable",
    TH_RUNTIME_ERROR: "RuntimeError",
}

# Every exported symbol of include/tilers_hip.h with (restype, argtypes).
_vp = C.c_void_p
_u32 = C.c_uint32
_u64 = C.c_uint64
_sz = C.c_size_t
_i = C.c_int
_cp = C.c_char_p
_f = C.c_float
_pp = C.POINTER(C.c_void_p)
_ppc = C.POINTER(C.c_char_p)


class EmitOpts(C.Structure):
    _fields_ = [("ub_size", C.c_size_t)]


EMIT_FN = C.CFUNCTYPE(C.c_int, C.c_char_p, C.c_size_t, C.POINTER(EmitOpts), _ppc, _ppc, _ppc, _ppc)

SIGNATURES: dict[str, tuple] = {
    "th_last_error": (_cp, []),
    "th_version": (_cp, []),
    "th_backend_is_hip": (_i, [_cp]),
    "th_backend_from_env": (_i, []),
    "th_device_count": (_i, [C.POINTER(C.c_int)]),
    "th_device_open": (_i, [_u32, _pp]),
    "th_device_close": (_i, [_vp]),
    "th_device_ordinal": (_u32, [_vp]),
    "th_device_name": (_i, [_vp, C.c_char_p, _sz]),
    "th_device_arch": (_i, [_vp, C.c_char_p, _sz]),
    "th_mem_info": (_i, [_vp, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "th_device_cu_count": (_i, [_vp, C.POINTER(C.c_int)]),
    "th_stream_create": (_i, [_vp, _pp]),
    "th_stream_destroy": (_i, [_vp]),
    "th_stream_sync": (_i, [_vp]),
    "th_malloc": (_i, [_vp, _sz, _pp]),
    "th_free": (_i, [_vp, _vp]),
    "th_memcpy_htod_async": (_i, [_vp, _vp, _sz, _vp]),
    "th_memcpy_dtoh_async": (_i, [_vp, _vp, _sz, _vp]),
    "th_memcpy_htod": (_i, [_vp, _vp, _sz]),
    "th_memcpy_dtoh": (_i, [_vp, _vp, _sz]),
    "th_memcpy_dtod_async": (_i, [_vp, _vp, _sz, _vp]),
    "th_memset_async": (_i, [_vp, _i, _sz, _vp]),
    "th_event_create": (_i, [_pp]),
    "th_event_destroy": (_i, [_vp]),
    "th_event_record": (_i, [_vp, _vp]),
    "th_event_sync": (_i, [_vp]),
    "th_event_elapsed_ms": (_i, [_vp, _vp, C.POINTER(C.c_float)]),
    "th_launcher_create": (_i, [_vp, _pp]),
    "th_launcher_destroy": (_i, [_vp]),
    "th_launcher_load": (_i, [_vp, _cp, _i]),
    "th_launcher_launch": (_i, [_vp, _cp, _u32, _u32, _u32, _pp, _sz, _vp]),
    "th_launcher_grid": (_i, [_vp, _cp, _u32, _pp, _sz, C.POINTER(C.c_uint64), C.POINTER(C.c_uint32)]),
    "th_softmax": (_i, [_vp, _vp, _u32, _u32, _i, _vp]),
    "th_matmul": (_i, [_vp, _vp, _vp, _u32, _u32, _u32, _i, _i, _i, _u32, _u64, _u64, _u64, _vp]),
    "th_matmul_silu_mul": (_i, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _i, _i, _i, _u32, _u64, _u64,
                                _u64, _vp]),
    "th_rms_norm": (_i, [_vp, _vp, _u32, _u32, _f, _i, _vp]),
    "th_causal_mask_f32": (_i, [_vp, _vp, _u32, _u32, _u32, _vp]),
    "th_attention": (_i, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _i, _vp]),
    "th_attention_prefill": (_i, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                                  _i, _vp]),
    "th_attention_decode_workspace_size": (_sz, [_u32, _u32, _u32, _u32, _u32]),
    "th_attention_decode": (_i, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _i, _vp,
                                 _sz, _vp]),
    "th_attention_decode_static": (_i, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32,
                                        _i, _vp]),
    "th_fill_random": (_i, [_vp, _u64, _i, _i, _f, _f, _u64, _vp]),
    "th_target_name": (_cp, []),
    "th_emit": (_i, [_cp, _sz, C.POINTER(EmitOpts), _ppc, _ppc, _ppc, _ppc]),
    "th_string_free": (None, [_vp]),
    "th_compile": (_i, [_cp, _sz, _cp, _cp, _ppc]),
    "th_registry_new": (_vp, []),
    "th_registry_with_builtin": (_vp, []),
    "th_registry_free": (None, [_vp]),
    "th_registry_register": (_i, [_vp, _cp, _cp, EMIT_FN]),
    "th_registry_len": (_sz, [_vp]),
    "th_registry_names": (_sz, [_vp, _ppc, _sz]),
    "th_registry_emit": (_i, [_vp, _cp, _cp, _sz, C.POINTER(EmitOpts), _ppc, _ppc, _ppc, _ppc]),
}

_LIB = None


class HalError(Exception):
    """Mirror of tile_hal's HalError (crates/tile_hal/src/error.rs:5-35)."""

    def __init__(self, code: int, message: str):
        self.code = code
        self.kind = ERROR_KINDS.get(code, "RuntimeError")
        super().__init__(message)

    def __str__(self) -> str:  # Display impl: "<category>: <message>"
        prefix = {
            "DeviceError": "device error",
            "MemoryError": "memory error",
            "KernelError": "kernel error",
            "StreamError": "stream error",
            "BackendNotAvailable": "backend not available",
            "RuntimeError": "runtime error",
        }[self.kind]
        return f"{prefix}: {self.args[0]}"


def load(path: Path | None = None):
    """Load (once) and declare the library.  Raises HalError when it is missing."""
    global _LIB
    if _LIB is not None:
        return _LIB
    p = Path(path) if path else library_path()
    if not p.exists():
        raise HalError(TH_BACKEND_NOT_AVAILABLE,
                       f"{p} is not built; run __graft_entry__.build() first")
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError:
            continue  # reported by missing_symbols(); calling it raises AttributeError
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def missing_symbols() -> list:
    """Header symbols the loaded library does not export."""
    lib = load()
    out = []
    for name in SIGNATURES:
        try:
            getattr(lib, name)
        except AttributeError:
            out.append(name)
    return out


def check(rc: int) -> None:
    if rc != TH_OK:
        msg = load().th_last_error().decode(errors="replace")
        raise HalError(rc, msg)

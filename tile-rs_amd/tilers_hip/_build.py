"""Build libtilers_hip.so (gfx950) in-tree from tile-rs_amd/csrc.

HIP translation units go through hipcc for gfx950 only; the codegen-target C++
(MLIR parser, emitter, registry) has no device code and goes through g++.
Objects are compiled in parallel and linked into
tile-rs_amd/tilers_hip/lib/libtilers_hip.so, which travels with the tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import hashlib
import math
import os
import re
import shutil
import subprocess
import tempfile
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent                      # tile-rs_amd/
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
LIB_DIR = PKG_DIR / "lib"
OBJ_DIR = ROOT / "_build"
LIB_NAME = "libtilers_hip.so"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

# Packed-FP32 instructions are disabled for every device compile (they have
# produced wrong results on this hardware pool); hipcc -O3 would otherwise
# form them from ordinary float code.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wno-unused-command-line-argument",
]
HOST_CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra"]

HIP_SOURCES = ["ops.hip", "ops_gemm.hip", "runtime.cpp"]
CPP_SOURCES = ["target/mlir_parse.cpp", "target/emit_hip.cpp", "target/registry.cpp"]


# A compiler diagnostic that is an error here: an asm statement that clobbers
# registers the function does not own (the register file split that the AGPR
# form of the prefill loop caused) is undefined behaviour on the GPU.
_FATAL_WARNINGS = ("clobber list contains reserved registers",)


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}")
    for w in _FATAL_WARNINGS:
        if w in proc.stdout:
            raise RuntimeError(f"build step warned '{w}': {' '.join(cmd)}\n{proc.stdout}")


# ---------------------------------------------------------------------------
# Source stamp: every built artefact carries the hash of the sources it was
# built from, so a run can tell whether the code it loads is the tree's.
# ---------------------------------------------------------------------------
STAMP_SUFFIXES = (".hip", ".cpp", ".hpp", ".h", ".inc", ".py", ".mlir")
STAMP_TAG = b"th-src:"


def _stamp_files() -> list[Path]:
    roots = (CSRC, INCLUDE, PKG_DIR / "examples")
    files = [p for r in roots for p in r.rglob("*")
             if p.is_file() and p.suffix in STAMP_SUFFIXES and "__pycache__" not in p.parts]
    files += [REF_MLIR_DIR / f"{stem}.mlir" for stem in REF_HOT_PATH]
    return sorted(files, key=lambda p: p.relative_to(ROOT.parent).as_posix())


def source_stamp() -> str:
    """First 16 hex digits of a SHA-256 over csrc/ (kernels, emitter, runtime, the
    prefill and GEMM generators and their generated includes), include/, the example MLIR and
    the reference's hot-path MLIR test inputs that are compiled for the GPU tests."""
    h = hashlib.sha256()
    for p in _stamp_files():
        data = p.read_bytes()
        h.update(p.relative_to(ROOT.parent).as_posix().encode() + b"\0")
        h.update(len(data).to_bytes(8, "little") + data)
    return h.hexdigest()[:16]


def stamp_define(stamp: str) -> list[str]:
    return [f'-DTH_BUILD_STAMP="{stamp}"']


def code_object_stamp(path: Path) -> str | None:
    """The stamp embedded in a built code object or library (None when absent)."""
    m = re.search(re.escape(STAMP_TAG) + rb"([0-9a-f]{16}|unstamped)", Path(path).read_bytes())
    return m.group(1).decode() if m else None


# ---------------------------------------------------------------------------
# Register and LDS budget of every kernel in a built code object.  A workgroup
# of W threads puts ceil(W/64) waves on the CU's four SIMDs; each SIMD lane has
# 512 unified VGPR+AGPR registers (allocated in granules of 8) and the CU has
# 160 KB of LDS.  A kernel whose descriptor asks for more cannot be dispatched:
# the command processor rejects the packet (ROCr reports it as
# HSA_STATUS_ERROR_INVALID_ISA and aborts the queue).
# ---------------------------------------------------------------------------
LLVM_BIN = ROCM / "llvm" / "bin"
UNIFIED_REGS_PER_LANE = 512
LDS_BYTES_PER_CU = 160 * 1024
BUNDLE_TARGET = f"hipv4-amdgcn-amd-amdhsa--{ARCH}"


def kernel_metadata(code_object: Path) -> list[dict]:
    """Per-kernel fields of the AMDGPU metadata note of a gfx950 ELF code object."""
    import yaml
    out = subprocess.run([str(LLVM_BIN / "llvm-readelf"), "--notes", str(code_object)],
                         stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, check=True)
    text = out.stdout
    start = text.find("---")
    end = text.find("...", start)
    meta = yaml.safe_load(text[start:end if end > 0 else None])
    return meta.get("amdhsa.kernels", [])


def _device_objects(path: Path, work: Path) -> list[Path]:
    """The gfx950 ELF code objects inside a --genco bundle or a hipcc -c object."""
    bundle = work / (path.name + ".bundle")
    if path.suffix == ".o":
        _run([str(LLVM_BIN / "llvm-objcopy"), f"--dump-section=.hip_fatbin={bundle}", str(path),
              str(work / (path.name + ".discard"))])
    else:
        shutil.copyfile(path, bundle)
    co = work / (path.name + ".co")
    _run([str(LLVM_BIN / "clang-offload-bundler"), "--unbundle", "--type=o",
          f"--input={bundle}", f"--targets={BUNDLE_TARGET}", f"--output={co}"])
    return [co]


def budget_violations(meta: list[dict]) -> list[str]:
    bad = []
    for k in meta:
        w = int(k.get(".max_flat_workgroup_size", 1024))
        per_simd = math.ceil(math.ceil(w / 64) / 4)
        regs = int(k.get(".vgpr_count", 0))   # unified count: arch VGPRs + AGPRs
        need = math.ceil(regs / 8) * 8 * per_simd
        if need > UNIFIED_REGS_PER_LANE:
            bad.append(f"{k.get('.name')}: {regs} unified registers x {per_simd} waves per SIMD "
                       f"({w}-thread workgroups) > {UNIFIED_REGS_PER_LANE}")
        lds = int(k.get(".group_segment_fixed_size", 0))
        if lds > LDS_BYTES_PER_CU:
            bad.append(f"{k.get('.name')}: {lds} B of LDS > {LDS_BYTES_PER_CU}")
    return bad


def check_code_objects(paths) -> None:
    """Raise if any kernel of the given built objects cannot be dispatched."""
    bad = []
    with tempfile.TemporaryDirectory() as d:
        for p in paths:
            for co in _device_objects(Path(p), Path(d)):
                bad += [f"{Path(p).name}: {b}" for b in budget_violations(kernel_metadata(co))]
    if bad:
        raise RuntimeError("kernels over the gfx950 register/LDS budget:\n  " + "\n  ".join(bad))


def _compile_hip(src: Path, obj: Path, stamp: str) -> None:
    lang = ["-x", "hip"] if src.suffix == ".hip" else ["-D__HIP_PLATFORM_AMD__"]
    _run([HIPCC, *DEVICE_FLAGS, *stamp_define(stamp), *lang, "-I", str(CSRC), "-I", str(INCLUDE),
          "-c", str(src), "-o", str(obj)])


def _compile_cpp(src: Path, obj: Path, stamp: str) -> None:
    cxx = shutil.which("g++") or "g++"
    _run([cxx, *HOST_CXX_FLAGS, *stamp_define(stamp), "-I", str(CSRC), "-I", str(INCLUDE), "-c",
          str(src), "-o", str(obj)])


EXAMPLES_DIR = PKG_DIR / "examples"
EXAMPLES_OUT = LIB_DIR / "examples"

# The reference's own MLIR test inputs for the tile ops of this path (stored as data
# under tests/golden/ref_mlir by tests/golden/extract_ref_mlir.py): the linalg
# bridge's MATMUL, SOFTMAX, ATTENTION, ATTENTION_DECODE_KERNEL, RMS_NORM and
# ATTN_PREFILL_MLIR constants (mlir_to_linalg.rs:1941, :1957, :2088, :2550, :2629,
# :2978) and the gpu emitter's softmax, matmul_f16 and attention_gqa tests
# (mlir_to_gpu.rs:2185, :2612, :2995).  Each is emitted by the hip target and
# compiled like the examples, so the GPU tests run them against the oracle.
REF_MLIR_DIR = ROOT.parent / "tests" / "golden" / "ref_mlir"
REF_OUT = LIB_DIR / "ref_fixtures"
REF_HOT_PATH = (
    "linalg__matmul", "linalg__softmax", "linalg__attention", "linalg__attention_decode_kernel",
    "linalg__rms_norm", "linalg__attn_prefill_mlir", "gpu__softmax_mlir_0",
    "gpu__matmul_f16_mlir_0", "gpu__attention_gqa_mlir_0",
)


def library_path() -> Path:
    return LIB_DIR / LIB_NAME


def example_path(stem: str) -> Path:
    return EXAMPLES_OUT / f"{stem}.hsaco"


def ref_fixture_path(stem: str) -> Path:
    return REF_OUT / f"{stem}.hsaco"


def build_examples(verbose: bool = False) -> list:
    """Emit every tilers_hip/examples/*.mlir, and the reference's hot-path MLIR test
    inputs, through the hip target and compile the HIP source into
    lib/examples/<stem>.hsaco and lib/ref_fixtures/<stem>.hsaco (the code objects
    the launcher loads)."""
    import importlib

    lib = importlib.import_module("tilers_hip")
    stamp = source_stamp()
    EXAMPLES_OUT.mkdir(parents=True, exist_ok=True)
    REF_OUT.mkdir(parents=True, exist_ok=True)
    srcs = []
    for mlir in sorted(EXAMPLES_DIR.glob("*.mlir")):
        out = lib.emit(mlir.read_text())
        hip = EXAMPLES_OUT / f"{mlir.stem}.hip"
        hip.write_text(out.source)
        srcs.append((hip, example_path(mlir.stem)))
    for stem in REF_HOT_PATH:
        out = lib.emit((REF_MLIR_DIR / f"{stem}.mlir").read_text())
        hip = REF_OUT / f"{stem}.hip"
        hip.write_text(out.source)
        srcs.append((hip, ref_fixture_path(stem)))

    def one(pair):
        hip, hsaco = pair
        _run([HIPCC, "--genco", *DEVICE_FLAGS, *stamp_define(stamp), "-I", str(CSRC), str(hip),
              "-o", str(hsaco)])
        return hsaco

    workers = max(1, min(len(srcs), os.cpu_count() or 1, 16))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        built = list(ex.map(one, srcs))
    check_code_objects(built)
    if verbose:
        print(f"built {len(built)} code objects in {EXAMPLES_OUT} and {REF_OUT}")
    return built


GENERATED = [
    # (generator script, output) -- generated device code included by ops.hip and ops_gemm.hip
    (CSRC / "kernels" / "gen_prefill.py", CSRC / "kernels" / "gen" / "prefill_asm.inc"),
    (CSRC / "kernels" / "gen_gemm.py", CSRC / "kernels" / "gen" / "gemm_asm.inc"),
]


def generate() -> None:
    """Run the code generators (they rewrite their output only when it changes)."""
    import sys
    for script, out in GENERATED:
        _run([sys.executable, str(script), str(out)])


def build(verbose: bool = False) -> Path:
    """Compile every source and link the shared library; returns its path."""
    generate()
    stamp = source_stamp()
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    jobs = []
    objs = []
    for rel in HIP_SOURCES:
        src = CSRC / rel
        obj = OBJ_DIR / (rel.replace("/", "_") + ".o")
        jobs.append((_compile_hip, src, obj))
        objs.append(obj)
    for rel in CPP_SOURCES:
        src = CSRC / rel
        if not src.exists():
            continue
        obj = OBJ_DIR / (rel.replace("/", "_") + ".o")
        jobs.append((_compile_cpp, src, obj))
        objs.append(obj)
    workers = max(1, min(len(jobs), os.cpu_count() or 1, 16))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        futs = [ex.submit(fn, src, obj, stamp) for fn, src, obj in jobs]
        for f in futs:
            f.result()
    check_code_objects([OBJ_DIR / (rel.replace("/", "_") + ".o") for rel in HIP_SOURCES
                        if rel.endswith(".hip")])
    out = library_path()
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp),
          "-Wl,-soname," + LIB_NAME, "-ldl"])
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    build_examples(verbose)
    return out


if __name__ == "__main__":
    import sys
    sys.path.insert(0, str(ROOT))
    build(verbose=True)

"""Build libtilers_hip.so (gfx950) in-tree from tile-rs_amd/csrc.

HIP translation units go through hipcc for gfx950 only; the codegen-target C++
(MLIR parser, emitter, registry) has no device code and goes through g++.
Objects are compiled in parallel and linked into
tile-rs_amd/tilers_hip/lib/libtilers_hip.so, which travels with the tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
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

HIP_SOURCES = ["ops.hip", "runtime.cpp"]
CPP_SOURCES = ["target/mlir_parse.cpp", "target/emit_hip.cpp", "target/registry.cpp"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}")


def _compile_hip(src: Path, obj: Path) -> None:
    lang = ["-x", "hip"] if src.suffix == ".hip" else ["-D__HIP_PLATFORM_AMD__"]
    _run([HIPCC, *DEVICE_FLAGS, *lang, "-I", str(CSRC), "-I", str(INCLUDE), "-c", str(src),
          "-o", str(obj)])


def _compile_cpp(src: Path, obj: Path) -> None:
    cxx = shutil.which("g++") or "g++"
    _run([cxx, *HOST_CXX_FLAGS, "-I", str(CSRC), "-I", str(INCLUDE), "-c", str(src),
          "-o", str(obj)])


EXAMPLES_DIR = PKG_DIR / "examples"
EXAMPLES_OUT = LIB_DIR / "examples"


def library_path() -> Path:
    return LIB_DIR / LIB_NAME


def example_path(stem: str) -> Path:
    return EXAMPLES_OUT / f"{stem}.hsaco"


def build_examples(verbose: bool = False) -> list:
    """Emit every tilers_hip/examples/*.mlir through the hip target and compile the
    HIP source into lib/examples/<stem>.hsaco (the code objects the launcher loads)."""
    import ctypes as C
    import importlib

    lib = importlib.import_module("tilers_hip")
    EXAMPLES_OUT.mkdir(parents=True, exist_ok=True)
    srcs = []
    for mlir in sorted(EXAMPLES_DIR.glob("*.mlir")):
        out = lib.emit(mlir.read_text())
        hip = EXAMPLES_OUT / f"{mlir.stem}.hip"
        hip.write_text(out.source)
        srcs.append((hip, example_path(mlir.stem)))

    def one(pair):
        hip, hsaco = pair
        _run([HIPCC, "--genco", *DEVICE_FLAGS, "-I", str(CSRC), str(hip), "-o", str(hsaco)])
        return hsaco

    workers = max(1, min(len(srcs), os.cpu_count() or 1, 16))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        built = list(ex.map(one, srcs))
    if verbose:
        print(f"built {len(built)} example code objects in {EXAMPLES_OUT}")
    return built


GENERATED = [
    # (generator script, output) -- generated device code included by ops.hip
    (CSRC / "kernels" / "gen_prefill.py", CSRC / "kernels" / "gen" / "prefill_asm.inc"),
]


def generate() -> None:
    """Run the code generators (they rewrite their output only when it changes)."""
    import sys
    for script, out in GENERATED:
        _run([sys.executable, str(script), str(out)])


def build(verbose: bool = False) -> Path:
    """Compile every source and link the shared library; returns its path."""
    generate()
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
        futs = [ex.submit(fn, src, obj) for fn, src, obj in jobs]
        for f in futs:
            f.result()
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

"""Extract the reference's own MLIR test inputs into text fixtures.

The reference keeps its codegen test inputs as raw-string constants in its Rust
sources: mlir_to_linalg.rs (tests module, :1912-2990), mlir_to_gpu.rs (tests,
:2102-2165) and tile_spec/tests/cucumber.rs (:97-234).  This script copies those
MLIR strings (test inputs, i.e. data) into tests/golden/ref_mlir/<origin>__<name>.mlir
so that the emitter's tests can run them without /root/reference.  Run it in a
container that has the reference mounted:

    python tests/golden/extract_ref_mlir.py [/root/reference]
"""
from __future__ import annotations

import re
import sys
from pathlib import Path

OUT = Path(__file__).resolve().parent / "ref_mlir"
SOURCES = {
    "linalg": "crates/rustc_codegen_tile/src/mlir_to_linalg.rs",
    "gpu": "crates/rustc_codegen_tile/src/mlir_to_gpu.rs",
    "cucumber": "crates/tile_spec/tests/cucumber.rs",
}
CONST = re.compile(r'const\s+([A-Z0-9_]+)\s*:\s*&str\s*=\s*r#"(.*?)"#;', re.S)
INLINE = re.compile(r'fn\s+([a-z0-9_]+)\s*\(\)[^{]*\{(.*?)\n    \}', re.S)
RAW = re.compile(r'r#"(.*?)"#', re.S)


def extract(root: Path) -> dict[str, str]:
    found: dict[str, str] = {}
    for origin, rel in SOURCES.items():
        text = (root / rel).read_text()
        for name, body in CONST.findall(text):
            if "module" in body and "llvm.func" in body:
                found[f"{origin}__{name.lower()}"] = body.strip() + "\n"
        if origin == "gpu":
            # the gpu emitter's tests pass their inputs inline to test functions
            tests = text[text.index("#[cfg(test)]"):]
            for fn, body in INLINE.findall(tests):
                for i, raw in enumerate(RAW.findall(body)):
                    if "module" in raw and "llvm.func" in raw:
                        found[f"{origin}__{fn}_{i}"] = raw.strip() + "\n"
    return found


def main() -> None:
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    OUT.mkdir(parents=True, exist_ok=True)
    found = extract(root)
    for old in OUT.glob("*.mlir"):
        old.unlink()
    for name, body in sorted(found.items()):
        (OUT / f"{name}.mlir").write_text(body)
    print(f"{len(found)} fixtures -> {OUT}")


if __name__ == "__main__":
    main()

"""The C ABI library loads and exports every symbol include/tilers_hip.h declares;
host-only entry points behave like their tile_hal counterparts.  No GPU needed
(no compute call is made)."""
from __future__ import annotations

import re
from pathlib import Path

import pytest

import tilers_hip as th
from tilers_hip import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "tilers_hip.h"


def header_symbols() -> set:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(th_[a-z0-9_]+)\s*\(", text)) - {"th_emit_fn"}


def test_header_symbols_are_declared_in_binding():
    assert header_symbols() == set(_lib.SIGNATURES)


def test_library_exports_every_header_symbol():
    _lib.load()
    assert _lib.missing_symbols() == []


def test_version_and_target_name():
    assert "gfx950" in th.lib().th_version().decode()
    assert th.target_name() == "hip"


def test_backend_selection(monkeypatch):
    # BackendKind::from_codegen_path (crates/tile_hal/src/backend.rs:27-40) + the hip arm
    assert th.BackendSelector.from_codegen_path("hip") is th.BackendKind.Hip
    assert th.BackendSelector.from_codegen_path("gpu") is None
    monkeypatch.setenv("TILERS_CODEGEN_PATH", "hip")
    assert th.BackendSelector.from_env().kind() is th.BackendKind.Hip
    monkeypatch.setenv("TILERS_CODEGEN_PATH", "nonsense")
    with pytest.raises(th.HalError) as e:
        th.BackendSelector.from_env()
    assert e.value.kind == "BackendNotAvailable" and "nonsense" in str(e.value)
    assert str(e.value).startswith("backend not available: unknown codegen path")
    monkeypatch.delenv("TILERS_CODEGEN_PATH")
    monkeypatch.setenv("ACLRS_CODEGEN_PATH", "hip")  # legacy name (backend.rs:72)
    assert th.BackendSelector.from_env().kind() is th.BackendKind.Hip
    monkeypatch.delenv("ACLRS_CODEGEN_PATH")
    with pytest.raises(th.HalError):  # default "cpp" is not this backend
        th.BackendSelector.from_env()


def test_launch_grid_builders():
    g = th.LaunchGrid.cuda(8192, 256).with_shared_mem(1024)
    assert (g.blocks, g.threads_per_block, g.shared_mem_bytes) == (8192, 256, 1024)
    assert th.LaunchGrid.blocks_only(4) == th.LaunchGrid(4, 1, 0)


def test_hal_error_display():
    e = th.HalError(_lib.TH_KERNEL_ERROR, "launch failed")
    assert str(e) == "kernel error: launch failed" and e.kind == "KernelError"

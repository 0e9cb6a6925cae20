"""Shared test setup.

`-m "not gpu"` tests run anywhere (oracle pinning, host logic, ABI exports).
`-m gpu` tests need an MI355X; they call the HIP path through the C ABI and
compare it with the CPU oracle.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "tile-rs_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def golden():
    def _load(name: str):
        return np.load(GOLDEN / name, allow_pickle=False)
    return _load


@pytest.fixture(scope="session")
def dev():
    import tilers_hip as th
    d = th.HipDevice(0)
    yield d


@pytest.fixture(scope="session")
def stream(dev):
    s = dev.create_stream()
    yield s
    s.synchronize()

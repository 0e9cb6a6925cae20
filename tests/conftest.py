"""Shared test setup.

`-m "not gpu"` tests run anywhere (oracle pinning, host logic, ABI exports).
`-m gpu` tests need an MI355X; they call the HIP path through the C ABI and
compare it with the CPU oracle.
"""
from __future__ import annotations

import sys
from pathlib import Path
from types import SimpleNamespace

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


CONFIG4_SEEDS = (0x71130000 + 4, 0x71130000 + 104, 0x71130000 + 204)


@pytest.fixture(scope="session")
def config4(dev, stream):
    """BASELINE config 4 (causal attention, B=4 H=32 S=4096 D=128 bf16) on the device
    PRNG with bench.py's seeds, and the oracle's output for every query row of every
    (batch, head), computed once per session and shared by the library and emitted
    tests."""
    import tilers_hip as th
    from oracle import oracle as orc
    B, H, S, Dh = 4, 32, 4096, 128
    n = B * S * H * Dh
    bufs = []
    for seed in CONFIG4_SEEDS:
        b = dev.alloc(n, th.TileDtype.BF16)
        th.fill_random(b, n, th.TileDtype.BF16, "normal", 0.0, 1.0, seed, stream)
        bufs.append(b)
    q, k, v = (b.copy_to_host(stream) for b in bufs)
    ref = orc.attention_prefill(q, k, v, orc.BF16, B, S, 0, S, Dh, H, H).reshape(B, S, H, Dh)
    return SimpleNamespace(B=B, H=H, S=S, Dh=Dh, n=n, q=bufs[0], k=bufs[1], v=bufs[2], ref=ref)

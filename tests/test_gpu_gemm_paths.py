"""The whole-tile GEMM's two kernels give the same bits (MI355X only).

Whole 256 x 256 tiles run on the generated-assembly program; TILERS_HIP_GEMM_ASM=0 (read
by the library on every call) sends them to the LDS-DMA kernel.  Both accumulate K in
the same order, so C must match bit for bit on random (not integer-valued) operands.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import tilers_hip as th

pytestmark = pytest.mark.gpu

D = th.TileDtype

# enough tiles (more than half the CUs) that neither run splits K
CASES = [(4096, 512, 4096, D.BF16, D.F32, False), (2048, 1024, 4608, D.F16, D.F16, False),
         (4096, 512, 2304, D.BF16, D.BF16, True)]


@pytest.mark.parametrize("m,k,n,ind,outd,bt", CASES)
def test_assembly_and_dma_kernels_agree_bitwise(dev, stream, m, k, n, ind, outd, bt):
    print(f"gemm paths {m}x{k}x{n} {ind}->{outd} bt={bt}", flush=True)
    a, b = dev.alloc(m * k, ind), dev.alloc(k * n, ind)
    th.fill_random(a, m * k, ind, "normal", 0.0, 1.0, 0x5eed01, stream)
    th.fill_random(b, k * n, ind, "normal", 0.0, 0.05, 0x5eed02, stream)
    out = {}
    for asm in ("1", "0"):
        c = dev.alloc(m * n, outd)
        old = os.environ.get("TILERS_HIP_GEMM_ASM")
        os.environ["TILERS_HIP_GEMM_ASM"] = asm
        try:
            th.matmul(a, b, c, m, k, n, ind, outd, bt, stream=stream)
        finally:
            if old is None:
                del os.environ["TILERS_HIP_GEMM_ASM"]
            else:
                os.environ["TILERS_HIP_GEMM_ASM"] = old
        out[asm] = c.copy_to_host(stream)
    got, ref = out["1"], out["0"]
    assert np.array_equal(got.view(np.uint8), ref.view(np.uint8)), \
        f"{int((got != ref).sum())} elements differ"

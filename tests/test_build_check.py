"""Build provenance and dispatchability of the built code objects.

Every artefact the build writes carries a stamp (a hash of csrc/, include/ and
the example MLIR; tilers_hip/_build.py source_stamp), so a run can show that the
code it loads was built from the tree it runs in.  The build also reads the
AMDGPU metadata of every kernel and rejects one that asks for more unified
VGPR+AGPR registers or LDS than its workgroup size allows: such a dispatch is
refused by the command processor and ROCr aborts the queue with
HSA_STATUS_ERROR_INVALID_ISA.  That is how an emitted prefill kernel built
against an AGPR form of the generated loop (264 registers at 512 threads per
workgroup) once aborted, while the library kernel with the same loop fit.
"""
from __future__ import annotations

from pathlib import Path

import pytest

import tilers_hip as th
from tilers_hip import _build

EXAMPLES = sorted(p.stem for p in _build.EXAMPLES_DIR.glob("*.mlir"))


def _check_stamps():
    want = _build.source_stamp()
    ver = th.lib().th_version().decode()
    assert ver.endswith("th-src:" + want), (ver, want)
    assert _build.code_object_stamp(_build.library_path()) == want
    for stem in EXAMPLES:
        assert _build.code_object_stamp(_build.example_path(stem)) == want, stem
    for stem in _build.REF_HOT_PATH:
        assert _build.code_object_stamp(_build.ref_fixture_path(stem)) == want, stem


def test_built_artefacts_carry_the_tree_stamp():
    _check_stamps()


@pytest.mark.gpu
def test_gpu_box_runs_the_tree_it_holds():
    """The same check on the GPU box, before any GPU test runs kernels."""
    _check_stamps()


def test_stamp_changes_with_any_source(tmp_path, monkeypatch):
    before = _build.source_stamp()
    files = _build._stamp_files()
    assert any(p.name == "prefill_asm.inc" for p in files)
    assert any(p.name == "gen_prefill.py" for p in files)
    assert any(p.suffix == ".mlir" for p in files)
    # a copy of the tree with one byte of the generated include changed stamps differently
    inc = next(p for p in files if p.name == "prefill_asm.inc")
    data = bytearray(inc.read_bytes())
    data[-2] ^= 1
    real_read = Path.read_bytes

    def fake_read(self):
        return bytes(data) if self == inc else real_read(self)

    monkeypatch.setattr(Path, "read_bytes", fake_read)
    assert _build.source_stamp() != before


def test_budget_rule():
    ok = [{".name": "k", ".max_flat_workgroup_size": 512, ".vgpr_count": 256,
           ".group_segment_fixed_size": 163840}]
    assert _build.budget_violations(ok) == []
    # the aborted dispatch: 192 arch VGPRs + 72 AGPRs at 512 threads
    agpr = [{".name": "prefill_bf16", ".max_flat_workgroup_size": 512, ".vgpr_count": 264,
             ".agpr_count": 72, ".group_segment_fixed_size": 163840}]
    assert "264 unified registers" in _build.budget_violations(agpr)[0]
    # one wave per SIMD may use all 512
    assert _build.budget_violations([{".name": "k", ".max_flat_workgroup_size": 256,
                                      ".vgpr_count": 512}]) == []
    assert _build.budget_violations([{".name": "k", ".max_flat_workgroup_size": 1024,
                                      ".vgpr_count": 136}])   # 4 waves per SIMD x 136 > 512
    assert _build.budget_violations([{".name": "k", ".max_flat_workgroup_size": 64,
                                      ".group_segment_fixed_size": 163841}])


def test_every_built_kernel_fits_its_workgroup():
    objs = [_build.example_path(s) for s in EXAMPLES]
    for name in ("ops.hip.o", "ops_gemm.hip.o"):
        if (_build.OBJ_DIR / name).exists():
            objs.append(_build.OBJ_DIR / name)
    _build.check_code_objects(objs)


_OVER_BUDGET = r'''
#include <hip/hip_runtime.h>
extern "C" __global__ void __launch_bounds__(512, 1) over(float* p) {
  float x = p[threadIdx.x];
  asm volatile("v_mov_b32 v250, %0\n\tv_accvgpr_write_b32 a60, v250" : : "v"(x)
               : "v250", "a60", "a61", "a62", "a63", "a64", "a65", "a66", "a67");
  p[threadIdx.x] = x;
}
'''


def test_build_rejects_an_asm_statement_over_the_register_budget(tmp_path):
    """An asm statement that names AGPRs on top of high VGPRs in a 512-thread kernel is
    refused by the build (compiler diagnostic or the metadata budget), never shipped."""
    src = tmp_path / "over.hip"
    src.write_text(_OVER_BUDGET)
    out = tmp_path / "over.hsaco"
    with pytest.raises(RuntimeError, match="reserved registers|register/LDS budget"):
        _build._run([_build.HIPCC, "--genco", *_build.DEVICE_FLAGS, str(src), "-o", str(out)])
        _build.check_code_objects([out])

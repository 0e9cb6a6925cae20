"""The `hip` CodegenTarget and the TargetRegistry (CPU only).

Mirrors the reference's registry/trait tests (crates/tile_codegen/src/lib.rs:
69-148) and its behaviour specs (crates/tile_spec/features/
backend_emit_purity.feature, core_op_lowering.feature,
registry_add_target.feature): empty-module rejection, byte-identical re-emit,
per-op lowering, and adding a target by registration.
"""
from __future__ import annotations

from pathlib import Path

import pytest

import tilers_hip as th
from tilers_hip import _build

EXAMPLES = Path(_build.EXAMPLES_DIR)


def mlir_one(op_line: str, loads: int = 1, store: str = "__tile_store_f32",
             load: str = "__tile_load_f32", name: str = "k", rows: int = 1, cols: int = 1024,
             extra_consts: str = "") -> str:
    args = ", ".join(f"%arg{i}: !llvm.ptr<1>" for i in range(loads + 1))
    body = [f"    %r = llvm.mlir.constant({rows} : i32) : i32",
            f"    %c = llvm.mlir.constant({cols} : i32) : i32", extra_consts]
    for i in range(loads):
        body.append(f"    %t{i} = llvm.call @{load}(%arg{i}, %r, %c) : (!llvm.ptr<1>, i32, i32) -> i32")
    body.append(op_line)
    body.append(f"    llvm.call @{store}(%arg{loads}, %y, %r, %c) : (!llvm.ptr<1>, i32, i32, i32) -> ()")
    body.append("    llvm.return")
    return ("module {\n  llvm.func @" + name + "(" + args + ") attributes {hacc.entry} {\n    ^bb0:\n"
            + "\n".join(l for l in body if l) + "\n  }\n}\n")


# ---- registry (crates/tile_codegen/src/lib.rs:69-148) ---------------------------------

def test_builtin_registry_has_debug_and_hip():
    r = th.TargetRegistry.with_builtin()
    assert r.names() == ["debug", "hip"]
    assert len(r) == 2 and not r.is_empty()
    assert r.select("hip").name() == "hip"
    assert r.select("cuda") is None
    assert th.TargetRegistry.new().is_empty()


def test_debug_target_echoes_module():
    r = th.TargetRegistry.with_builtin()
    out = r.select("debug").emit("func.func @a\nfunc.func @b\n")
    assert out.source == "// tile-rs debug target\n// 2 MLIR lines, 2 func.func op(s)\nfunc.func @a\nfunc.func @b\n\n"
    assert out.ext == "mlir.txt"


@pytest.mark.parametrize("target", ["debug", "hip"])
def test_empty_module_is_an_error(target):
    r = th.TargetRegistry.with_builtin()
    with pytest.raises(th.HalError) as e:
        r.select(target).emit("   \n ")
    assert "empty MLIR module" in str(e.value)


def test_module_without_entry_kernel_is_an_error():
    src = mlir_one("    %y = llvm.call @__tile_softmax_f32(%t0, %t0, %r, %c) : (i32, i32, i32, i32) -> i32")
    with pytest.raises(th.HalError) as e:
        th.emit(src.replace("attributes {hacc.entry}", ""))
    assert "No entry-point kernel functions" in str(e.value)


def test_register_custom_target_and_select_by_codegen_path(monkeypatch):
    # registry_add_target.feature: register a target, select it by TILERS_CODEGEN_PATH
    r = th.TargetRegistry.with_builtin()
    r.register(th.EmitterTarget("myaccel", "acc", lambda m: "// myaccel\n" + m))
    monkeypatch.setenv("TILERS_CODEGEN_PATH", "myaccel")
    import os
    t = r.select(os.environ["TILERS_CODEGEN_PATH"])
    out = t.emit("x")
    assert out.source == "// myaccel\nx" and out.ext == "acc"
    r.register(th.EmitterTarget("failing", "x", lambda m: (_ for _ in ()).throw(ValueError("nope"))))
    with pytest.raises(th.HalError) as e:
        r.select("failing").emit("x")
    assert "nope" in str(e.value)


def test_select_returns_first_registered_of_a_name():
    r = th.TargetRegistry.new()
    r.register(th.EmitterTarget("dup", "a", lambda m: "first"))
    r.register(th.EmitterTarget("dup", "b", lambda m: "second"))
    assert r.select("dup").emit("x").source == "first"


# ---- hip target: purity and lowering -------------------------------------------------------

@pytest.mark.parametrize("path", sorted(EXAMPLES.glob("*.mlir")), ids=lambda p: p.stem)
def test_emit_is_deterministic(path):
    text = path.read_text()
    a, b = th.emit(text), th.emit(text)
    assert a.source == b.source and a.ext == "hip" and a.meta == b.meta
    assert a.meta.kernel_names and not a.meta.has_cube_kernel
    for name in a.meta.kernel_names:
        assert f'extern "C" __global__' in a.source and f"__th_desc_{name}" in a.source


def test_registry_hip_matches_direct_emit():
    text = (EXAMPLES / "softmax_rows.mlir").read_text()
    assert th.TargetRegistry.with_builtin().select("hip").emit(text).source == th.emit(text).source


@pytest.mark.parametrize("example,entry", [
    ("softmax_rows", "th::entry::softmax_rows<th::kF32, 4>"),
    ("softmax_generic", "th::entry::softmax_rows<th::kBF16, 4>"),
    ("matmul_bf16", "th::entry::gemm_dma<th::kBF16, th::kF32, false, th::gemm::kEpiStore>"),
    ("matmul_f16_t", "th::entry::gemm_dma<th::kF16, th::kF16, true, th::gemm::kEpiStore>"),
    ("matmul_f32", "th::entry::gemm_f32<th::kF32, false, true, th::gemm::kEpiStore>"),
    ("attention_f32", "th::entry::attention_tiles<th::kF32, 256>"),
    ("prefill_bf16", "th::entry::prefill<th::kBF16>"),
    ("decode_bf16", "th::entry::decode<th::kBF16>"),
    ("rms_norm_rows", "th::entry::rms_norm_rows<th::kF32, 4>"),
    ("swiglu_gate_bf16", "th::entry::gemm_dma<th::kBF16, th::kF32, false, th::gemm::kEpiSiluMul>"),
    ("matmul_bf16_tiles", "th::entry::gemm_dma<th::kBF16, th::kBF16, false, th::gemm::kEpiStore>"),
])
def test_hot_ops_lower_to_hand_written_kernels(example, entry):
    out = th.emit((EXAMPLES / f"{example}.mlir").read_text())
    assert entry in out.source


def test_matmul_launch_shapes_follow_the_entry():
    """K a multiple of 32: the LDS-DMA entry, 512-thread workgroups, one per started
    256x256 tile (512x320x768: 2 x 3; 512x256x384: 2 x 2).  Other 16-bit K: the
    register-staged entry with 256 threads."""
    src = th.emit((EXAMPLES / "matmul_bf16_tiles.mlir").read_text()).source
    assert "__launch_bounds__(512) matmul_bf16_tiles(" in src
    assert "__th_desc_matmul_bf16_tiles = {th::kLaunchDescMagic, 512u, 6u, 1u," in src
    src = th.emit((EXAMPLES / "matmul_bf16.mlir").read_text()).source
    assert "__launch_bounds__(512) matmul_bf16_acc_f32(" in src
    assert "__th_desc_matmul_bf16_acc_f32 = {th::kLaunchDescMagic, 512u, 4u, 1u," in src
    k96 = (EXAMPLES / "matmul_bf16.mlir").read_text().replace("constant(256 : i32)",
                                                                "constant(96 : i32)")
    src = th.emit(k96).source
    assert "__launch_bounds__(512) matmul_bf16_acc_f32(" in src
    k72 = (EXAMPLES / "matmul_bf16.mlir").read_text().replace("constant(256 : i32)",
                                                                "constant(72 : i32)")
    src = th.emit(k72).source
    assert "th::entry::gemm<th::kBF16, th::kF32, false, th::gemm::kEpiStore>" in src
    assert "__launch_bounds__(256) matmul_bf16_acc_f32(" in src


def test_whole_tile_matmuls_lower_to_the_assembly_entry():
    """The config GEMMs (4096^3 bf16 -> f32; 8192x4096x14336 f16 -> f16): whole 256x256
    tiles, row-major B, K a multiple of 128 -> the generated-assembly entry, 256-thread
    workgroups (one per CU), one per tile.  A K of 96 or an N of 384 keeps the DMA entry."""
    src = th.emit((EXAMPLES / "config_gemms.mlir").read_text()).source
    assert "th::entry::gemm_asm<th::kBF16, th::kF32, false>(" in src
    assert "th::entry::gemm_asm<th::kF16, th::kF16, false>(" in src
    assert "__launch_bounds__(256, 1) gemm_4096_bf16_acc_f32(" in src
    assert "__th_desc_gemm_4096_bf16_acc_f32 = {th::kLaunchDescMagic, 256u, 256u, 1u," in src
    assert "__th_desc_mlp_up_f16 = {th::kLaunchDescMagic, 256u, 1792u, 1u," in src
    gate = src[src.index("kernel mlp_gate_f16"):]
    assert "th::entry::gemm_asm<th::kF16, th::kF16, false, true>(" in gate
    assert "__th_desc_mlp_gate_f16 = {th::kLaunchDescMagic, 256u, 1792u, 1u," in gate
    assert "th::entry::gemm_dma" not in src
    k96 = (EXAMPLES / "matmul_bf16.mlir").read_text().replace("constant(256 : i32)",
                                                                "constant(96 : i32)")
    assert "th::entry::gemm_dma<" in th.emit(k96).source
    # B stored N x K on whole tiles: the same entry's transposed program
    t = (EXAMPLES / "matmul_f16_t.mlir").read_text()
    for old, new in (("128 : i32", "256 : i32"), ("320 : i32", "512 : i32"),
                     ("264 : i32", "768 : i32")):
        t = t.replace(f"constant({old})", f"constant({new})")
    assert "th::entry::gemm_asm<th::kF16, th::kF16, true>(" in th.emit(t).source


def test_matmul_shape_and_tile_offsets_are_exact():
    out = th.emit((EXAMPLES / "matmul_bf16.mlir").read_text())
    # M=512 K=256 N=384: th::entry::gemm_dma(..., M, N, K, tiles); 2 x 2 workgroups per tile
    assert "512u, 384u, 256u, th_tiles" in out.source
    assert "__th_desc_matmul_bf16_acc_f32 = {th::kLaunchDescMagic, 512u, 4u, 1u" in out.source


def test_attention_runtime_params_follow_metal_order():
    pre = th.emit((EXAMPLES / "prefill_bf16.mlir").read_text()).source
    assert ("uint32_t seq_len, uint32_t start_pos, uint32_t max_seq, uint32_t head_dim, "
            "uint32_t num_heads, uint32_t num_kv_heads, uint32_t th_tiles") in pre
    dec = th.emit((EXAMPLES / "decode_bf16.mlir").read_text()).source
    assert ("uint32_t seq_len, uint32_t max_seq, uint32_t head_dim, uint32_t num_heads, "
            "uint32_t num_kv_heads, uint32_t th_tiles") in dec


def test_elementwise_fallback():
    out = th.emit((EXAMPLES / "swiglu_mask.mlir").read_text())
    assert out.meta.kernel_names == ["swiglu", "scaled_causal"]
    assert "/ (1.0f + expf(-" in out.source            # silu
    assert "(col <= row ?" in out.source                 # causal mask: keep col <= row
    assert "0x1p-3f" in out.source                       # scale 0.125, exact
    assert "th::minimumf(th::maximumf(" in out.source    # clamp: NaN-propagating min/max


def test_long_rows_lower_to_one_workgroup_per_row():
    src = th.emit((EXAMPLES / "rows_long.mlir").read_text()).source
    assert "th::entry::softmax_rows_wg<th::kF32, 16>(" in src      # 4096 vectors per row
    assert "__th_desc_softmax_long_f32 = {th::kLaunchDescMagic, 256u, 1u, 1u," in src
    assert "th::entry::rms_norm_rows_wg<th::kF32, 8>(" in src      # 2048 vectors per row
    assert "__th_desc_rms_long_f32 = {th::kLaunchDescMagic, 256u, 2u, 1u," in src


def test_rope_lowers_to_pair_rotation():
    out = th.emit((EXAMPLES / "rope.mlir").read_text())
    assert out.meta.kernel_names == ["rope_f32", "rope_bf16"]
    src = out.source
    # freq = 1 / 10000^(2j / cols) in f32, angle = pos * freq (mlir_to_gpu.rs:1536-1545)
    assert "1.0f / powf(10000.0f, 2.0f * static_cast<float>(col >> 1) / 0x1p+6f)" in src
    assert "0x1.cp+2f * r" in src                       # pos 7, exact
    assert "0x1.f4p+9f * r" in src                      # pos 1000, exact
    assert "static_cast<int64_t>(i ^ 1ull)" in src       # the pair partner
    assert "th::u16_to_f32<th::kBF16>" in src            # bf16 side channel from the name


def test_rope_needs_even_cols_and_a_loaded_input():
    rope = ("    %p = llvm.mlir.constant(3 : i32) : i32\n"
            "    %y = llvm.call @__tile_rope_f32(%t0, %t0, %p, %r, %c) : (i32, i32, i32, i32, i32) -> i32")
    with pytest.raises(th.HalError) as e:
        th.emit(mlir_one(rope, cols=63))
    assert "cols must be even" in str(e.value)
    chained = ("    %e = llvm.call @__tile_exp_f32(%t0, %t0, %r, %c) : (i32, i32, i32, i32) -> i32\n"
               "    %p = llvm.mlir.constant(3 : i32) : i32\n"
               "    %y = llvm.call @__tile_rope_f32(%e, %e, %p, %r, %c) : (i32, i32, i32, i32, i32) -> i32")
    with pytest.raises(th.HalError) as e:
        th.emit(mlir_one(chained))
    assert "rope input must come straight from a load" in str(e.value)


# The core tile-op set every open backend lowers (tile_spec/features/
# core_op_lowering.feature:8-41), as rows for the hip target.
@pytest.mark.parametrize("op,evidence", [
    ("rms_norm", "th::entry::rms_norm_rows"),
    ("matmul", "th::entry::gemm"),
    ("softmax", "th::entry::softmax_rows"),
    ("rope", "cosf("),
    ("add", " + "),
])
def test_core_op_lowers_to_hip(op, evidence):
    lines = {
        "rms_norm": ("    %e = llvm.mlir.constant(0 : i32) : i32\n"
                     "    %y = llvm.call @__tile_rms_norm_f32(%e, %t0, %e, %r, %c) : (i32, i32, i32, i32, i32) -> i32", 1),
        "softmax": ("    %y = llvm.call @__tile_softmax_f32(%t0, %t0, %r, %c) : (i32, i32, i32, i32) -> i32", 1),
        "rope": ("    %p = llvm.mlir.constant(7 : i32) : i32\n"
                 "    %y = llvm.call @__tile_rope_f32(%t0, %t0, %p, %r, %c) : (i32, i32, i32, i32, i32) -> i32", 1),
        "add": ("    %y = llvm.call @__tile_add_f32(%t0, %t0, %t1, %r, %c) : (i32, i32, i32, i32, i32) -> i32", 2),
    }
    if op == "matmul":
        text = (EXAMPLES / "matmul_f16_t.mlir").read_text()
    else:
        line, loads = lines[op]
        text = mlir_one(line, loads=loads, rows=4, cols=256, name=f"{op}_k")
    out = th.emit(text)
    assert evidence in out.source
    assert th.emit(text).source == out.source  # pure: byte-identical on re-emit


def test_bf16_side_channel_from_names():
    body = "    %y = llvm.call @__tile_softmax_f16(%t0, %t0, %r, %c) : (i32, i32, i32, i32) -> i32"
    f16 = th.emit(mlir_one(body, load="__tile_load_f16", store="__tile_store_f16", name="sm"))
    assert "th::kF16" in f16.source and "th::kBF16" not in f16.source
    bf = th.emit(mlir_one(body, load="__tile_load_f16", store="__tile_store_f16", name="sm_bf16"))
    assert "th::kBF16" in bf.source
    explicit = th.emit(mlir_one(body, load="__tile_load_bf16", store="__tile_store_bf16", name="sm"))
    assert "th::kBF16" in explicit.source


def test_generic_form_matches_pretty_form():
    gen = th.emit((EXAMPLES / "softmax_generic.mlir").read_text())
    assert gen.meta.kernel_names == ["softmax_bf16_generic"]
    assert "th_tiles * 4u, 2048u" in gen.source


def test_unsupported_intrinsic_is_an_error():
    body = "    %y = llvm.call @__tile_topk_f32(%t0, %t0, %r, %c) : (i32, i32, i32, i32) -> i32"
    with pytest.raises(th.HalError) as e:
        th.emit(mlir_one(body))
    assert "unsupported intrinsic __tile_topk_f32" in str(e.value)
    assert e.value.kind == "KernelError"


def test_hot_op_must_be_fed_by_loads():
    body = ("    %e = llvm.call @__tile_exp_f32(%t0, %t0, %r, %c) : (i32, i32, i32, i32) -> i32\n"
            "    %y = llvm.call @__tile_softmax_f32(%e, %e, %r, %c) : (i32, i32, i32, i32) -> i32")
    with pytest.raises(th.HalError) as e:
        th.emit(mlir_one(body))
    assert "operands must come straight from loads" in str(e.value)


def test_constant_gep_offsets_are_applied():
    src = mlir_one("    %y = llvm.call @__tile_softmax_f32(%t0, %t0, %r, %c) : (i32, i32, i32, i32) -> i32")
    src = src.replace("    %t0 = llvm.call @__tile_load_f32(%arg0,",
                      "    %o = llvm.mlir.constant(4096 : i64) : i64\n"
                      "    %p = llvm.getelementptr %arg0[%o] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, f32\n"
                      "    %t0 = llvm.call @__tile_load_f32(%p,")
    out = th.emit(src)
    assert "(reinterpret_cast<const float*>(p0) + 4096ll)" in out.source


def test_emitted_module_compiles_for_gfx950(tmp_path):
    out = th.emit((EXAMPLES / "swiglu_mask.mlir").read_text())
    co = tmp_path / "swiglu.hsaco"
    th.compile_source(out.source, co)
    assert co.stat().st_size > 1000


def test_compile_error_is_reported(tmp_path):
    with pytest.raises(th.HalError) as e:
        th.compile_source("this is not C++", tmp_path / "bad.hsaco")
    assert "hipcc failed" in str(e.value)


def test_rms_norm_eps_and_shape_are_exact():
    out = th.emit((EXAMPLES / "rms_norm_rows.mlir").read_text()).source
    # eps constant 9.99999997E-7 is the f32 nearest 1e-6, printed exactly
    assert "th_tiles * 4u, 768u, 0x1.0c6f7ap-20f)" in out


def test_fused_swiglu_takes_up_from_its_own_view():
    out = th.emit((EXAMPLES / "swiglu_gate_bf16.mlir").read_text()).source
    # C = silu(X.W) * U: A = p0, B = p1, C = p3, UP = p2 (f32, the output dtype)
    assert ("(reinterpret_cast<float*>(p3)), 256u, 256u, 512u, th_tiles, "
            "(reinterpret_cast<const float*>(p2)));") in out
    assert "silu*mul epilogue" in out


def test_fused_swiglu_whole_tiles_16bit_lower_to_the_assembly_entry():
    out = th.emit((EXAMPLES / "swiglu_gate_bf16.mlir").read_text()).source
    fn = out[out.index("kernel swiglu_gate_f16"):]
    assert "th::entry::gemm_asm<th::kF16, th::kF16, false, true>(" in fn
    assert ("(reinterpret_cast<uint16_t*>(p3)), 256u, 512u, 512u, th_tiles, "
            "(reinterpret_cast<const uint16_t*>(p2)));") in fn
    assert "__launch_bounds__(256, 1) swiglu_gate_f16" in fn


def test_fused_swiglu_rejects_up_in_another_dtype():
    text = (EXAMPLES / "swiglu_gate_bf16.mlir").read_text().replace(
        "%u = llvm.call @__tile_load_f32(%arg2", "%u = llvm.call @__tile_load_f16(%arg2")
    with pytest.raises(th.HalError, match="UP in the output dtype"):
        th.emit(text)


def test_silu_mul_without_matmul_stays_elementwise():
    out = th.emit((EXAMPLES / "swiglu_mask.mlir").read_text()).source
    assert "elementwise" in out and "kEpiSiluMul" not in out


# ---- the reference's own MLIR test inputs (tests/golden/ref_mlir, extracted by
#      tests/golden/extract_ref_mlir.py from mlir_to_linalg.rs:1912-2990,
#      mlir_to_gpu.rs tests and tile_spec/tests/cucumber.rs:97-234) ----------------------

REF_MLIR = Path(__file__).resolve().parent / "golden" / "ref_mlir"
# Model-level ops outside the tile-op hot path (sampling, speculative decoding,
# gather/scatter, int8 quantization, KV-cache writes, rope variants): the hip target
# rejects them with an explicit error.
REF_REJECTED = {
    "cucumber__sample_top_p_mlir", "cucumber__token_accept_mlir",
    "gpu__concat_mlir_0", "gpu__gather_mlir_0", "gpu__scatter_mlir_0", "gpu__slice_mlir_0",
    "gpu__test_gpu_draft_verify_0", "gpu__test_gpu_sample_top_p_0", "gpu__test_gpu_token_accept_0",
    "gpu__topk_mlir_0", "linalg__dequant_mlir", "linalg__kv_cache_update_kernel",
    "linalg__kvup_prefill_mlir", "linalg__quant_mlir", "linalg__rope_inplace_kernel",
    "linalg__rope_prefill_mlir", "linalg__sample_top_p",
}


def _ref_fixtures():
    return sorted(REF_MLIR.glob("*.mlir"))


def test_reference_fixtures_are_present():
    names = {p.stem for p in _ref_fixtures()}
    assert len(names) == 87
    assert REF_REJECTED <= names


@pytest.mark.parametrize("path", _ref_fixtures(), ids=lambda p: p.stem)
def test_reference_fixture_through_hip_target(path):
    text = path.read_text()
    if path.stem in REF_REJECTED:
        with pytest.raises(th.HalError) as e:
            th.emit(text)
        assert "unsupported intrinsic" in str(e.value)
        return
    out = th.emit(text)
    assert out.ext == "hip" and "extern \"C\" __global__" in out.source
    assert th.emit(text).source == out.source   # deterministic


def test_attention_gqa_lowers_to_the_head_major_prefill():
    """__tile_attention_gqa_* (the gpu emitter's causal GQA attention with head-major
    Q/O, mlir_to_gpu.rs:1627-1712): the prefill entry in its head-major form, sizes
    from the intrinsic's constant operands."""
    src = th.emit((REF_MLIR / "gpu__attention_gqa_mlir_0.mlir").read_text()).source
    assert "th::entry::prefill<th::kF32, true>(" in src
    assert "th_tiles, 32u, 0u, 32u, 64u, 8u, 2u);" in src
    # f32: one workgroup per (head, query)
    assert "__th_desc_tile_attention_gqa = {th::kLaunchDescMagic, 512u, 256u, 1u," in src
    ex = th.emit((EXAMPLES / "attention_gqa.mlir").read_text()).source
    # bf16 with head_dim 128: the MFMA kernel, one workgroup per (head, 256 queries)
    assert "th::entry::prefill<th::kBF16, true>(" in ex and "th_tiles, 300u, 0u, 300u, 128u, 8u, 2u);" in ex
    assert "__th_desc_attention_gqa_bf16 = {th::kLaunchDescMagic, 512u, 16u, 1u," in ex
    bad = (REF_MLIR / "gpu__attention_gqa_mlir_0.mlir").read_text().replace(
        "constant(2 : i32) : i32\n    %seq", "constant(3 : i32) : i32\n    %seq")
    with pytest.raises(th.HalError, match="multiple of num_kv_heads"):
        th.emit(bad)


def test_new_ops_lower_to_their_entries():
    out = th.emit((EXAMPLES / "ops_extra.mlir").read_text())
    src = out.source
    for evidence in ("logf(", "tanhf(", "fabsf(", "(1.0f / sqrtf(", "(1.0f / (expf(-", "th::minimumf(", "th::maximumf(",
                     "th::entry::reduce_rows<th::entry::kRowSum>", "kRowMax>", "kRowAbsMax>",
                     "kRowArgMax>", "th::entry::transpose(", "th::entry::matvec("):
        assert evidence in src, evidence
    # reduction outputs: one value per row, the stored view of tile t at t * rows
    assert "th_tiles, 8u, 1000u, 8ull);" in src
    assert "th_tiles, 96u, 200u, 200ull, 96ull);" in src


# ---- counted tile loops and the pipelined_for marker (tile.rs:2168-2221) --------------------

def loop_module(body: str, bound: str = "%arg2", pred: str = "uge", depth: int | None = 2,
                step: str = "%one", start: str = "%zero", cols: int = 1024, name: str = "lp",
                extra: str = "") -> str:
    """The loop of tile.rs:2196-2210 (`loop { if i >= n_tiles { break; } ... i += 1 }`)
    around a softmax over one 1 x `cols` row per iteration."""
    marker = ("    %depth = llvm.mlir.constant(" + str(depth) + " : i32) : i32\n"
              "    llvm.call @__tile_pipelined_for_begin(%depth) : (i32) -> ()\n") if depth else ""
    end = "    llvm.call @__tile_pipelined_for_end() : () -> ()\n" if depth else ""
    return ("module {\n  llvm.func @" + name + "(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: i32)"
            " attributes {hacc.entry} {\n    ^bb0:\n" + marker +
            "    %zero = llvm.mlir.constant(0 : i32) : i32\n"
            "    %one = llvm.mlir.constant(1 : i32) : i32\n"
            "    %two = llvm.mlir.constant(2 : i32) : i32\n"
            f"    %cols = llvm.mlir.constant({cols} : i32) : i32\n"
            f"    %cols64 = llvm.mlir.constant({cols} : i64) : i64\n" + extra +
            f"    llvm.br ^bb1({start} : i32)\n"
            "  ^bb1(%i: i32):\n"
            f"    %done = llvm.icmp \"{pred}\" %i, {bound} : i32\n"
            "    llvm.cond_br %done, ^bb3, ^bb2\n"
            "  ^bb2:\n" + body +
            f"    %next = llvm.add %i, {step} : i32\n"
            "    llvm.br ^bb1(%next : i32)\n"
            "  ^bb3:\n" + end + "    llvm.return\n  }\n}\n")


LOOP_BODY = (
    "    %iw = llvm.zext %i : i32 to i64\n"
    "    %off = llvm.mul %iw, %cols64 : i64\n"
    "    %src = llvm.getelementptr %arg0[%off] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, f32\n"
    "    %dst = llvm.getelementptr %arg1[%off] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, f32\n"
    "    %t = llvm.call @__tile_load_f32(%src, %one, %cols) : (!llvm.ptr<1>, i32, i32) -> i32\n"
    "    %y = llvm.call @__tile_softmax_f32(%t, %t, %one, %cols) : (i32, i32, i32, i32) -> i32\n"
    "    llvm.call @__tile_store_f32(%dst, %y, %one, %cols) : (!llvm.ptr<1>, i32, i32, i32) -> ()\n")


def _shift_body(load_off: str, store_off: str) -> str:
    """A loop body that loads arg0 at `load_off` and stores arg0 at `store_off` (both i64
    SSA names defined in the body): a read and a write of the same buffer."""
    return ("    %iw = llvm.zext %i : i32 to i64\n"
            "    %off = llvm.mul %iw, %cols64 : i64\n"
            "    %one64 = llvm.mlir.constant(1 : i64) : i64\n"
            "    %ip = llvm.add %iw, %one64 : i64\n"
            "    %offp = llvm.mul %ip, %cols64 : i64\n"
            f"    %src = llvm.getelementptr %arg0[{load_off}] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, f32\n"
            f"    %dst = llvm.getelementptr %arg0[{store_off}] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, f32\n"
            "    %t = llvm.call @__tile_load_f32(%src, %one, %cols) : (!llvm.ptr<1>, i32, i32) -> i32\n"
            "    %y = llvm.call @__tile_softmax_f32(%t, %t, %one, %cols) : (i32, i32, i32, i32) -> i32\n"
            "    llvm.call @__tile_store_f32(%dst, %y, %one, %cols) : (!llvm.ptr<1>, i32, i32, i32) -> ()\n")


@pytest.mark.parametrize("load_off,store_off", [("%offp", "%off"), ("%off", "%offp")])
def test_loop_carried_dependence_is_rejected(load_off, store_off):
    """tile.rs:2187-2210 runs the loop body in order; the hip target runs iterations in
    parallel.  A loop that stores buffer p one tile behind (or ahead of) where it loads
    p has a loop-carried dependence, so parallel iterations would race: rejected."""
    with pytest.raises(th.HalError) as e:
        th.emit(loop_module(_shift_body(load_off, store_off)))
    assert "loop-carried dependence" in str(e.value)


def test_loop_in_place_update_is_lowered():
    """Loading and storing the same tile of one buffer (an in-place update) has no
    dependence between iterations."""
    src = th.emit(loop_module(_shift_body("%off", "%off"))).source
    assert "th::entry::softmax_rows<th::kF32, 4>(" in src


def test_loop_example_lowers_to_a_tile_grid():
    """The reference's loop example: iteration i becomes logical tile i, the trip count
    comes from the kernel's scalar argument and scales the grid through the descriptor
    (arg 2, ceil(n / 16) workgroups: 16 rows per workgroup)."""
    src = th.emit((EXAMPLES / "softmax_loop.mlir").read_text()).source
    assert ("softmax_loop_f32(void* __restrict__ p0, void* __restrict__ p1, uint32_t s2, "
            "uint32_t th_tiles_in)") in src
    assert "const uint32_t th_tiles = th_tiles_in ? s2 : 0u;" in src
    assert "th::entry::softmax_rows<th::kF32, 4>(" in src and "th_tiles * 1u, 1024u);" in src
    assert "__th_desc_softmax_loop_f32 = {th::kLaunchDescMagic, 256u, 1u, 1u, 0u, 3u, 16u, 65536u, 0u};" in src
    # an i64 bound (0x40 | 4 in the descriptor), `ult` with the body on the true edge,
    # `1 + i`, a shl-scaled offset
    assert "uint64_t s3, uint32_t th_tiles_in)" in src
    assert "th_tiles_in ? (s3 > 0xffffffffull ? 0xffffffffu : static_cast<uint32_t>(s3)) : 0u;" in src
    assert "__th_desc_add_loop_f32 = {th::kLaunchDescMagic, 256u, 2u, 1u, 0u, 68u, 1u, 65536u, 0u};" in src
    # a signed `i < n`: negative n is zero tiles, in the kernel and in the grid (0x80 | 3)
    assert "th_tiles_in ? (static_cast<int32_t>(s2) <= 0 ? 0u : s2) : 0u;" in src
    assert "__th_desc_softmax_loop_signed_f32 = {th::kLaunchDescMagic, 256u, 1u, 1u, 0u, 131u, 16u," in src


def test_loop_generic_form_and_constant_trip():
    src = th.emit((EXAMPLES / "softmax_loop_generic.mlir").read_text()).source
    assert "const uint32_t th_tiles = th_tiles_in ? 48u : 0u;" in src
    # 48 iterations of one 4-row tile, one workgroup each
    assert "__th_desc_softmax_loop_bf16_generic = {th::kLaunchDescMagic, 256u, 48u, 1u, 0u, 0u, 0u, 0u, 0u};" in src


def test_pipelined_for_marker_sets_the_pipeline_depth():
    """depth >= 2 keeps the next row in flight (streaming softmax); depth == 1 is the
    explicit opt-out (tile.rs:2179-2180); no marker behaves like depth 2."""
    two = th.emit(loop_module(LOOP_BODY, depth=2)).source
    one = th.emit(loop_module(LOOP_BODY, depth=1)).source
    none = th.emit(loop_module(LOOP_BODY, depth=None)).source
    assert "softmax_rows<th::kF32, 4>(" in two and "pipelined_for(2)" in two
    assert "softmax_rows<th::kF32, 4, false>(" in one and "pipelined_for(1)" in one
    assert "softmax_rows<th::kF32, 4>(" in none and "pipelined_for" not in none.split("->")[0]
    # 16 rows per streaming workgroup, 4 without streaming
    assert "0u, 3u, 16u, 65536u, 0u};" in two and "0u, 3u, 4u, 65536u, 0u};" in one


def test_pipelined_for_depth_is_the_gemm_lds_ring_depth():
    text = (EXAMPLES / "matmul_bf16.mlir").read_text()
    marker = ("    %pd = llvm.mlir.constant(5 : i32) : i32\n"
              "    llvm.call @__tile_pipelined_for_begin(%pd) : (i32) -> ()\n    %m =")
    src = th.emit(text.replace("    %m =", marker, 1)).source
    assert "th::entry::gemm_dma<th::kBF16, th::kF32, false, th::gemm::kEpiStore, 5>" in src
    plain = th.emit(text).source
    assert "th::entry::gemm_dma<th::kBF16, th::kF32, false, th::gemm::kEpiStore>" in plain


@pytest.mark.parametrize("mutate,message", [
    (dict(step="%two"), "the loop must step by 1"),
    (dict(start="%one"), "the loop must start at 0"),
    (dict(pred="ult"), "the loop must run while iv < n"),
    (dict(bound="%zero", body=LOOP_BODY.replace("%cols64 : i64", "%two64 : i64"),
          extra="    %two64 = llvm.mlir.constant(512 : i64) : i64\n"),
     "loop views must advance one tile"),
])
def test_loop_shapes_outside_the_counted_tile_loop_are_rejected(mutate, message):
    kw = dict(body=LOOP_BODY)
    kw.update(mutate)
    body = kw.pop("body")
    with pytest.raises(th.HalError) as e:
        th.emit(loop_module(body, **kw))
    assert message in str(e.value)


def test_signed_loop_bounds_run_no_iteration_when_negative():
    """`icmp sge %i, %n` (the loop of a signed `i >= n` test): a negative n runs no
    iteration, so the tile count is clamped at zero instead of wrapping to 2^32 - k."""
    src = th.emit(loop_module(LOOP_BODY, pred="sge")).source
    assert "th_tiles_in ? (static_cast<int32_t>(s2) <= 0 ? 0u : s2) : 0u;" in src
    neg = th.emit(loop_module(LOOP_BODY, pred="sge", bound="%neg",
                              extra="    %neg = llvm.mlir.constant(-5 : i32) : i32\n")).source
    assert "const uint32_t th_tiles = th_tiles_in ? 0u : 0u;" in neg
    # under an unsigned compare the same constant is 2^32 - 5 iterations: rejected
    with pytest.raises(th.HalError) as e:
        th.emit(loop_module(LOOP_BODY, pred="uge", bound="%neg",
                            extra="    %neg = llvm.mlir.constant(-5 : i32) : i32\n"))
    assert "negative trip count" in str(e.value)


def test_loop_bound_must_be_an_integer_argument():
    text = loop_module(LOOP_BODY).replace("%arg2: i32)", "%arg2: f32)")
    with pytest.raises(th.HalError) as e:
        th.emit(text)
    assert "must be an i32 or i64 argument" in str(e.value)


def test_loop_with_a_per_tile_offset_is_rejected():
    body = ("    %b = llvm.call @get_block_idx() : () -> i64\n"
            "    %bo = llvm.mul %b, %cols64 : i64\n"
            "    %a0 = llvm.getelementptr %arg0[%bo] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, f32\n"
            + LOOP_BODY.replace("%arg0[%off]", "%a0[%off]"))
    with pytest.raises(th.HalError) as e:
        th.emit(loop_module(body))
    assert "per-tile (block index) offset" in str(e.value)


def test_loop_compiles_for_gfx950(tmp_path):
    for stem in ("softmax_loop", "softmax_loop_generic"):
        co = tmp_path / f"{stem}.hsaco"
        th.compile_source(th.emit((EXAMPLES / f"{stem}.mlir").read_text()).source, co)
        assert co.stat().st_size > 1000


def test_loop_around_a_matmul_is_a_batched_gemm():
    src = th.emit((EXAMPLES / "gemm_loop.mlir").read_text()).source
    assert "th::entry::gemm_dma<th::kBF16, th::kF32, false, th::gemm::kEpiStore, 5>" in src
    assert "256u, 384u, 320u, th_tiles);" in src
    # two 256x256 output tiles per GEMM, times the trip count in argument 3
    assert "__th_desc_gemm_loop_bf16 = {th::kLaunchDescMagic, 512u, 2u, 1u, 0u, 4u, 1u, 65536u, 0u};" in src

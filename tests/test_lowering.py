"""Host-side lowering (no GPU): which gfx950 plan each tile program gets, and the epilogue chain the GEMM plan
carries to krn_gemm_nt."""

import math
from pathlib import Path
import pytest

from krn_amd.compiler import cdna4
from krn_amd.compiler.capture import capture
from tests.conftest import KERNELS

BASE = {"bm": 16, "bn": 16, "bk": 8, "bias": False, "relu": False, "gelu": False, "silu": False}
# reference src/krn/lib/lib_ours.py:38-46: the constants each lib.matmul epilogue sets
EPILOGUES = {
    "none": {}, "bias": {"bias": True}, "relu": {"relu": True}, "gelu": {"gelu": True},
    "bias_relu": {"bias": True, "relu": True}, "bias_gelu": {"bias": True, "gelu": True}, "silu": {"silu": True},
}  # fmt: skip


@pytest.mark.parametrize("name", list(EPILOGUES))
def test_lib_matmul_f16_lowers_to_the_mfma_gemm_with_its_epilogue(name):
    flags = EPILOGUES[name]
    plan = cdna4.lower(capture(KERNELS, "matmul_epilogue", consts={"t": {**BASE, **flags}}))
    assert isinstance(plan, cdna4.GemmPlan)
    assert plan.layout == "nn" and plan.c == "out"
    want = []
    if flags.get("bias"):
        want.append(("add", "bias", "col"))
    want += [(act, None, "") for act in ("relu", "gelu", "silu") if flags.get(act)]
    assert [(op.op, op.tensor, op.axis) for op in plan.ops] == want


def test_lib_matmul_f32_has_no_matrix_unit_product_and_lowers_generically():
    plan = cdna4.lower(capture(KERNELS, "matmul_epilogue_f32", consts={"t": {**BASE, "bias": True, "gelu": True}}))
    assert isinstance(plan, cdna4.GenericPlan)


@pytest.mark.parametrize("name, kind", [("gemm_nt", cdna4.GemmPlan), ("gemm_fp8", cdna4.GemmPlan),
                                        ("gemm_w8a8", cdna4.GemmPlan), ("gemm_i8_i32", cdna4.GemmPlan),
                                        ("matmul", cdna4.GemmPlan), ("row_softmax", cdna4.GenericPlan)])
def test_plan_kinds(name, kind):
    consts = {"t": {"bm": 64, "bn": 64, "bk": 32}} if kind is cdna4.GemmPlan else {"t": {"rows": 8, "cols": 16}}
    assert isinstance(cdna4.lower(capture(KERNELS, name, consts=consts)), kind)


def test_attention_program_lowers_to_the_attention_kernel():
    consts = {"t": {"bq": 64, "bk": 64, "d": 128, "causal": True}}
    kernel = capture(KERNELS, "flash_attention_bf16", consts=consts)
    plan = cdna4.lower(kernel)
    assert isinstance(plan, cdna4.AttentionPlan) and plan.d == 128 and plan.causal
    assert not any("flash-attention" in reason for reason in cdna4.why_generic(kernel))


def test_attention_the_kernel_does_not_serve_lowers_generically_and_says_why():
    """Head dimension 32 is outside the attention kernel: the program runs on the generic lowering, and the reason
    names the flash-attention match, so `explain()` reports the slower route instead of taking it silently."""
    kernel = capture(KERNELS, "flash_attention_bf16", consts={"t": {"bq": 64, "bk": 64, "d": 32, "causal": True}})
    assert isinstance(cdna4.lower(kernel), cdna4.GenericPlan)
    assert any("flash-attention" in reason for reason in cdna4.why_generic(kernel))



@pytest.mark.parametrize("name, long_rows, dtype", [
    ("softmax_long_rows", True, "f16"), ("softmax", False, "f16"), ("softmax_steps", False, "f16"),
    ("softmax_long_rows_bf16", True, "bf16"), ("softmax_bf16", False, "bf16"), ("softmax_f32", False, "f32"),
])  # fmt: skip
def test_softmax_programs_lower_to_the_row_softmax_kernel(name, long_rows, dtype):
    from krn_amd.dtypes import BF16, F16, F32

    dt = {"f16": F16, "bf16": BF16, "f32": F32}[dtype]
    plan = cdna4.lower(capture(KERNELS, name, consts={"t": {"rows": 4, "cols": 512}}))
    assert isinstance(plan, cdna4.SoftmaxPlan)
    assert (plan.x, plan.y, plan.dtype, plan.rows, plan.cols, plan.long_rows) == ("x", "y", dt, 4, 512, long_rows)


def test_a_softmax_over_fixed_rows_lowers_generically():
    """`row_softmax` reads rows 0..rows-1 in every block, not the block's own rows: not the kernel's function."""
    plan = cdna4.lower(capture(KERNELS, "row_softmax", consts={"t": {"rows": 4, "cols": 512}}))
    assert isinstance(plan, cdna4.GenericPlan)


def test_softmax_launch_passes_the_row_width_and_refuses_other_grids(monkeypatch):
    """Host side of the row-softmax launch: width min(cols, t.cols) for the one-tile forms and every column for the
    long-row form, one stride per row; a grid other than one block per t.rows rows, or x and y of different shapes,
    keeps the generic lowering."""
    from types import SimpleNamespace

    from krn_amd import Blocks
    from krn_amd.runtime import hip, library

    calls = []
    monkeypatch.setattr(library, "softmax_rows", lambda *a: calls.append(a))
    stream = SimpleNamespace(handle=7)
    for name, cols, width in [("softmax", 700, 512), ("softmax", 300, 300), ("softmax_long_rows", 3000, 3000)]:
        kernel = capture(KERNELS, name, consts={"t": {"rows": 4, "cols": 512}})
        plan = cdna4.lower(kernel)
        launch = hip.Launch(kernel, plan)
        x = SimpleNamespace(shape=(10, cols), pointer=100)
        y = SimpleNamespace(shape=(10, cols), pointer=200)
        params = {"x": x, "y": y}
        run = launch._softmax(plan, params, Blocks(3))
        run(stream)
        assert calls[-1][1:] == (100, 200, 10, width, cols, cols, 7)
        assert launch._softmax(plan, params, Blocks(4)) is None
        assert launch._softmax(plan, {"x": x, "y": SimpleNamespace(shape=(10, cols + 1), pointer=200)},
                               Blocks(3)) is None


def test_gemm_launch_marshals_once_and_refuses_partial_grids(monkeypatch):
    """The W8A8 program's launch: the row and column scale vectors become epilogue operations 1 and 2 (float32),
    the arguments are marshalled once at preparation, and a grid that does not cover the output keeps the generic
    lowering."""
    from types import SimpleNamespace

    from krn_amd import Blocks
    from krn_amd.dtypes import F32
    from krn_amd.runtime import hip, library

    made, ran = [], []

    def gemm_nt_call(*args):
        made.append(args)
        return lambda stream: ran.append(stream)

    monkeypatch.setattr(library, "gemm_nt_call", gemm_nt_call)
    kernel = capture(KERNELS, "gemm_w8a8", consts={"t": {"bm": 64, "bn": 64, "bk": 32}})
    plan = cdna4.lower(kernel)
    launch = hip.Launch(kernel, plan)
    m, n, k = 16, 200, 256
    params = {"a": SimpleNamespace(shape=(m, k), pointer=1), "w": SimpleNamespace(shape=(n, k), pointer=2),
              "scale_a": SimpleNamespace(shape=(m, 1), pointer=3, dtype=F32),
              "scale_w": SimpleNamespace(shape=(1, n), pointer=4, dtype=F32),
              "c": SimpleNamespace(shape=(m, n), pointer=5)}
    run = launch._gemm(plan, params, Blocks(4, 1))
    assert len(made) == 1
    _, a, b, c, _, mm, nn, kk, ops = made[0]
    assert (a, b, c, mm, nn, kk) == (1, 2, 5, m, n, k)
    assert ops == [(library.MUL_ROW, 0.0, 3), (library.MUL_COL, 0.0, 4)]
    for _ in range(3):
        run(SimpleNamespace(handle=9))
    assert ran == [9, 9, 9] and len(made) == 1
    assert launch._gemm(plan, params, Blocks(3, 1)) is None


@pytest.mark.parametrize("name, consts, products", [
    ("gemm_partial_k", {"bm": 64, "bn": 64, "bk": 32, "kk": 96}, ["mfma 16x16x32 bf16"]),
    ("gemm_partial_k", {"bm": 64, "bn": 64, "bk": 16, "kk": 96}, ["mfma 16x16x16 bf16"]),
    ("gemm_fp8", {"bm": 64, "bn": 64, "bk": 64}, ["mfma 16x16x32 fp8"]),
    ("gemm_i8_partial_k", {"bm": 64, "bn": 64, "bk": 64, "kk": 128}, ["mfma 16x16x32 i8"]),
    ("flash_attention_bf16", {"bq": 64, "bk": 64, "d": 32, "causal": True}, ["mfma 16x16x32 bf16"] * 2),
    ("flash_attention", {"bq": 8, "bk": 8, "d": 16, "causal": True}, ["scalar fma"] * 2),
    ("product", {"rows": 8, "cols": 16}, ["scalar fma"]),
])  # fmt: skip
def test_generic_products_take_the_matrix_cores_when_the_tile_extents_allow(name, consts, products):
    """m and n multiples of 16 and k of the instruction's K: a 16x16x16 f16/bf16 or 16x16x32 i8 MFMA; otherwise the
    scalar fused multiply-adds in k order."""
    from krn_amd.compiler import hipgen

    kernel = capture(KERNELS, name, consts={"t": consts})
    assert hipgen.products(kernel) == products
    source, _ = hipgen.emit(kernel, "krn_probe")
    assert ("__builtin_amdgcn_mfma" in source) == any(p.startswith("mfma") for p in products)


@pytest.mark.parametrize("name,consts,form", [
    ("gemm_i8_partial_k", {"bm": 64, "bn": 64, "bk": 64, "kk": 128}, "16x16x32 i8"),
    ("gemm_partial_k", {"bm": 64, "bn": 64, "bk": 32, "kk": 96}, "16x16x32 bf16"),
    ("gemm_fp8", {"bm": 64, "bn": 64, "bk": 64}, "16x16x32 fp8"),
    ("matmul", {"bm": 32, "bn": 32, "bk": 32}, "16x16x32 f16"),
    ("matmul", {"bm": 32, "bn": 32, "bk": 16}, "16x16x16 f16"),
])
def test_the_generic_mfma_source_compiles_for_gfx950(tmp_path, name, consts, form):
    """The generated products compile for gfx950 (hipcc cross-compiles here; the GPU tests run them)."""
    import shutil
    import subprocess

    from krn_amd.compiler import hipgen

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    kernel = capture(KERNELS, name, consts={"t": consts})
    assert hipgen.products(kernel) == [f"mfma {form}"]
    source, _ = hipgen.emit(kernel, "krn_probe")
    path = tmp_path / "probe.hip"
    path.write_text("#include <hip/hip_runtime.h>\n" + source)
    result = subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-c", str(path), "-o", str(tmp_path / "p.o")],
                            capture_output=True, text=True)
    assert result.returncode == 0, result.stderr[-2000:]


VARIANTS = Path(__file__).with_name("kernels") / "attention_variants.py"


@pytest.mark.parametrize("name,consts,want", [
    ("reordered", {"cfg": {"rows_per_block": 256, "keys_per_step": 32, "head_dim": 128, "masked": True}},
     {"q": "query", "k": "key", "v": "value", "o": "out", "bq": 256, "d": 128, "causal": True, "rank": 3}),
    ("reordered", {"cfg": {"rows_per_block": 64, "keys_per_step": 32, "head_dim": 64, "masked": False}},
     {"bq": 64, "d": 64, "causal": False, "base": 1.0}),
    ("natural_exp_4d", {"t": {"bq": 128, "bk": 64, "d": 128, "causal": True}},
     {"rank": 4, "causal": True, "base": math.log2(math.e)}),
])
def test_rewritten_attention_programs_are_recognised_by_their_dataflow(name, consts, want):
    """Other names, tilings, temporaries, operand orders, mask spellings, the natural exponential and 4-D
    (batch, heads, seq, d) indexing: the same online softmax, so the same hand-written kernel."""
    plan = cdna4.lower(capture(VARIANTS, name, consts=consts))
    assert isinstance(plan, cdna4.AttentionPlan)
    for field_name, value in want.items():
        assert getattr(plan, field_name) == value, field_name


@pytest.mark.parametrize("name", ["drifting", "unscaled_sum"])
def test_programs_that_compute_something_else_are_not_taken_for_attention(name):
    kernel = capture(VARIANTS, name, consts={"t": {"bq": 128, "bk": 64, "d": 128, "causal": True}})
    assert isinstance(cdna4.lower(kernel), cdna4.GenericPlan)
    assert any("flash-attention" in reason for reason in cdna4.why_generic(kernel))


SOFTMAXES = Path(__file__).with_name("kernels") / "softmax_variants.py"


@pytest.mark.parametrize("name,consts,long_rows", [
    ("running", {"cfg": {"per_block": 2, "chunk": 256}}, True),
    ("one_tile", {"cfg": {"per_block": 4, "width": 96}}, False),
])
def test_rewritten_softmax_programs_are_recognised_by_their_dataflow(name, consts, long_rows):
    plan = cdna4.lower(capture(SOFTMAXES, name, consts=consts))
    assert isinstance(plan, cdna4.SoftmaxPlan) and plan.long_rows == long_rows
    assert (plan.x, plan.y, plan.rows) == ("src", "dst", next(iter(consts.values()))["per_block"])


@pytest.mark.parametrize("name", ["unshifted", "reciprocal"])
def test_programs_that_round_differently_are_not_taken_for_the_softmax(name):
    kernel = capture(SOFTMAXES, name, consts={"cfg": {"per_block": 4, "width": 96}})
    assert isinstance(cdna4.lower(kernel), cdna4.GenericPlan)

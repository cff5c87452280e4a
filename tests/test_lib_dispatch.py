"""`lib.matmul`'s dispatcher on the host (no GPU): the reference's AMD order, refusals, declines and the generic
`matmul_epilogue` program's lowering for each element type."""

import pytest

from krn_amd.compiler import cdna4
from krn_amd.compiler.capture import CaptureError, capture
from krn_amd.dtypes import BF16, F16, F32, I8
from krn_amd.lib import kernels, lib


def problem(dtypes, epilogue=lib.Epilogue.NONE, shape=(4, 5, 6)):
    return lib.Problem(lib.Op.MATMUL, dtypes, shape, epilogue)


def test_the_amd_order_is_the_references():
    """reference src/krn/lib/lib.py:264: (Op.MATMUL, "amd"): ("hipblaslt", "ours", "host")"""
    assert lib.PREFERENCE[lib.Op.MATMUL] == ("hipblaslt", "ours", "host")


def test_refusals_name_each_candidate(monkeypatch):
    monkeypatch.delenv("KRN_LIB", raising=False)
    hip, ours, host = (lib.candidate(name) for name in lib.PREFERENCE[lib.Op.MATMUL])
    assert hip.refusal(problem((F16, F16, F16), lib.Epilogue.SILU)) is None
    assert "i8" in hip.refusal(problem((I8, I8, F32)))
    assert ours.refusal(problem((F16, F16, F32))) is not None and ours.refusal(problem((BF16,) * 3)) is None
    assert host.unavailable() is not None
    with pytest.raises(lib.NoCandidate):
        lib.choice(problem((I8, I8, F32)))


def test_a_declining_candidate_falls_to_the_next(monkeypatch):
    ran = []

    class Declines(lib.Candidate):
        name, op, origin = "hipblaslt", lib.Op.MATMUL, lib.Origin.VENDOR

        def refusal(self, p):
            return None

        def run(self, p, operands, stream):
            raise lib.Declined("no algorithm")

    class Runs(Declines):
        name = "ours"

        def run(self, p, operands, stream):
            ran.append(p)

    monkeypatch.setattr(lib, "candidate", {"hipblaslt": Declines(), "ours": Runs(), "host": lib.Host()}.get)
    monkeypatch.delenv("KRN_LIB", raising=False)
    assert lib.launch(problem((F16,) * 3), None, None) == "ours" and len(ran) == 1
    with pytest.raises(lib.NoCandidate, match="hipblaslt: no algorithm"):
        lib.launch(problem((F16,) * 3), None, None, library="hipblaslt")


def test_one_library_can_be_chosen(monkeypatch):
    monkeypatch.setenv("KRN_LIB", "ours")
    assert lib.order() == ("ours",)
    assert lib.order("hipblaslt") == ("hipblaslt",)
    monkeypatch.delenv("KRN_LIB")
    assert lib.order() == lib.PREFERENCE[lib.Op.MATMUL]


@pytest.mark.parametrize("dtype", [F16, BF16, F32])
def test_the_generic_matmul_program_takes_its_element_type_from_the_arguments(dtype):
    """`matmul_epilogue(..., a: Matrix[F], ...)` is generic over F (reference lib_kernels.py:31-34): 16-bit operands
    lower to the MFMA GEMM with the bias and GELU fused, f32 to the generic lowering."""
    consts = {"t": {"bm": 64, "bn": 64, "bk": 32, "bias": True, "relu": False, "gelu": True, "silu": False}}
    kernel = capture(kernels.__file__, "matmul_epilogue", consts=consts,
                     dtypes={name: dtype for name in ("a", "b", "bias", "out")})
    plan = cdna4.lower(kernel)
    if dtype == F32:
        assert isinstance(plan, cdna4.GenericPlan)
    else:
        assert isinstance(plan, cdna4.GemmPlan) and plan.operand == dtype and plan.layout == "nn"
        assert [(op.op, op.axis) for op in plan.ops] == [("add", "col"), ("gelu", "")]


def test_a_generic_tensor_needs_its_argument():
    with pytest.raises(CaptureError, match="generic over F"):
        capture(kernels.__file__, "matmul_epilogue", consts={"t": {"bm": 16, "bn": 16, "bk": 8}})


def test_a_bias_of_another_type_than_the_output_is_refused_before_anything_runs(monkeypatch):
    """The bias is a vector of the output type (reference lib.py:576-590 `bias: Vector[Y]`, `out: Matrix[Y]`).
    hipBLASLt reads it as the output type, so a mismatch is refused before any device call."""
    from types import SimpleNamespace

    def touched(*args, **kwargs):
        raise AssertionError("nothing may be allocated or launched")

    monkeypatch.setattr(lib, "default_device", touched)
    monkeypatch.setattr(lib, "launch", touched)
    a, b = SimpleNamespace(shape=(4, 6), dtype=BF16), SimpleNamespace(shape=(6, 5), dtype=BF16)
    out = SimpleNamespace(shape=(4, 5), dtype=F32)
    with pytest.raises(ValueError, match="needs a f32 bias"):
        lib.matmul(a, b, epilogue=lib.Epilogue.BIAS, bias=SimpleNamespace(shape=(5,), dtype=BF16), out=out)
    with pytest.raises(ValueError, match="needs a bf16 bias"):
        lib.matmul(a, b, epilogue="bias_gelu", bias=SimpleNamespace(shape=(5,), dtype=F32))


def test_epilogues_and_ops_compare_equal_to_their_names():
    """The reference's Epilogue and Op are StrEnums (lib.py:76-91)."""
    assert lib.Epilogue.BIAS_GELU == "bias_gelu" and lib.Epilogue("silu") is lib.Epilogue.SILU
    assert str(lib.Epilogue.RELU) == "relu" and lib.Op.MATMUL == "matmul"


def test_hipblaslt_plans_are_keyed_on_operand_alignment(monkeypatch):
    """An algorithm chosen for 256-byte aligned operands is not replayed on less aligned ones (reference
    lib_cublaslt.py:110-135 `PlanKey.alignments`)."""
    from types import SimpleNamespace

    from krn_amd.lib import lib_hipblaslt as lt

    made = []
    monkeypatch.setattr(lt, "Plan", lambda handle, problem: made.append(problem) or SimpleNamespace())
    session = lt.Session()
    session.handle = 1
    p = problem((BF16,) * 3)
    t = lambda pointer: SimpleNamespace(pointer=pointer)
    aligned = lib.Operands(t(0x10000), t(0x20000), t(0x30000), None)
    session.plan(p, aligned)
    session.plan(p, lib.Operands(t(0x40000), t(0x50100), t(0x60000), None))
    assert len(made) == 1  # 0x50100 is still 256-byte aligned
    session.plan(p, lib.Operands(t(0x40000), t(0x50002), t(0x60000), None))
    assert len(made) == 2
    assert lt.alignments(lib.Operands(t(0x50002), t(0x50040), t(0x1000), None)) == (2, 64, 256, 0)

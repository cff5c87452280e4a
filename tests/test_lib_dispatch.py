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

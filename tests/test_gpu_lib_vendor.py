"""`lib.matmul` on gfx950 through the reference's AMD candidate order (src/krn/lib/lib.py:264): hipBLASLt first,
then krn's own `matmul_epilogue` program. The hipBLASLt candidate is checked as the reference checks its vendor
adapters (tests/lib/test_lib_vendors.py:420-475): against float64 with a bound of 4 half-ulps of the output type times
the magnitude of the product (plus 2e-3 for the tanh-form GELU the vendor libraries compute), and against `ours`
within twice that (4e-3 for GELU, whose exact form krn's own program uses)."""

import math

import numpy as np
import pytest

from krn_amd import T
from krn_amd.dtypes import BF16, F16, F32
from krn_amd.lib import Epilogue, lib
from oracle.numerics import bf16_values, bf16_words

pytestmark = pytest.mark.gpu

TRIPLES = [(F16, F16, F16), (F16, F16, F32), (BF16, BF16, BF16), (BF16, BF16, F32), (F32, F32, F32)]
EPS = {F16: np.finfo(np.float16).eps, BF16: 2.0**-7, F32: np.finfo(np.float32).eps}


def upload(device, x: np.ndarray, dtype):
    if dtype == BF16:
        return device.to_device(bf16_words(x.astype(np.float32)), T.bf16)
    return device.to_device(x.astype(np.float16 if dtype == F16 else np.float32))


def host(x: np.ndarray, dtype) -> np.ndarray:
    """The values the device holds for `x` stored as `dtype`, as float64."""
    if dtype == BF16:
        return bf16_values(bf16_words(x.astype(np.float32))).astype(np.float64)
    return x.astype(np.float16 if dtype == F16 else np.float32).astype(np.float64)


def download(tensor, dtype) -> np.ndarray:
    got = tensor.to_host()
    return bf16_values(got).astype(np.float64) if dtype == BF16 else got.astype(np.float64)


def reference(a, b, bias, epilogue: Epilogue, exact_gelu: bool):
    x = a @ b
    magnitude = np.abs(a) @ np.abs(b)
    if epilogue.has_bias:
        x = x + bias
        magnitude = magnitude + np.abs(bias)
    if "relu" in epilogue.value:
        x = np.maximum(x, 0)
    if "gelu" in epilogue.value:
        if exact_gelu:
            x = 0.5 * x * (1 + np.vectorize(math.erf)(x / math.sqrt(2)))
        else:
            x = 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x**3)))
    if epilogue == Epilogue.SILU:
        x = x / (1 + np.exp(-x))
    return x, magnitude


def run(device, triple, shape, epilogue, library):
    m, n, k = shape
    rng = np.random.default_rng(31)
    a = rng.standard_normal((m, k)) / np.sqrt(k)
    b = rng.standard_normal((k, n))
    bias = rng.standard_normal(n)
    da, db, dbias = upload(device, a, triple[0]), upload(device, b, triple[1]), upload(device, bias, triple[2])
    out = device.empty(triple[2], m, n)
    lib.matmul(da, db, out=out, bias=dbias if epilogue.has_bias else None, epilogue=epilogue, library=library)
    return download(out, triple[2]), (host(a, triple[0]), host(b, triple[1]), host(bias, triple[2]))


@pytest.mark.parametrize("epilogue", list(Epilogue))
@pytest.mark.parametrize("triple", TRIPLES, ids=lambda t: "-".join(map(str, t)))
@pytest.mark.parametrize("shape", [(33, 29, 37), (1, 5, 3), (256, 384, 320)])
def test_hipblaslt_matmul(device, triple, shape, epilogue):
    problem = lib.Problem(lib.Op.MATMUL, triple, shape, epilogue)
    assert lib.choice(problem) == "hipblaslt"
    got, (a, b, bias) = run(device, triple, shape, epilogue, "hipblaslt")
    want, magnitude = reference(a, b, bias, epilogue, exact_gelu=False)
    bound = 4 * (EPS[triple[2]] / 2) * magnitude + (2e-3 if "gelu" in epilogue.value else 0)
    error = np.abs(got - want)
    assert np.all(error <= bound), f"max error {error.max()}, max excess {(error - bound).max()}"


@pytest.mark.parametrize("epilogue", list(Epilogue))
@pytest.mark.parametrize("triple", [(F16, F16, F16), (BF16, BF16, BF16), (F32, F32, F32)], ids=str)
def test_hipblaslt_agrees_with_ours(device, triple, epilogue):
    shape = (130, 257, 64)
    vendor, (a, b, bias) = run(device, triple, shape, epilogue, "hipblaslt")
    ours, _ = run(device, triple, shape, epilogue, "ours")
    _, magnitude = reference(a, b, bias, epilogue, exact_gelu=True)
    bound = 8 * (EPS[triple[2]] / 2) * magnitude + (4e-3 if "gelu" in epilogue.value else 0)
    assert np.all(np.abs(vendor - ours) <= bound)


def test_the_default_order_runs_hipblaslt_and_a_refused_problem_falls_to_ours(device):
    """int8 has no float hipBLASLt triple here: ours refuses it too, and the error lists each candidate's reason."""
    rng = np.random.default_rng(5)
    a = device.to_device(rng.uniform(-1, 1, (40, 24)).astype(np.float16))
    b = device.to_device(rng.uniform(-1, 1, (24, 56)).astype(np.float16))
    out = lib.matmul(a, b)
    want = a.to_host().astype(np.float64) @ b.to_host().astype(np.float64)
    np.testing.assert_allclose(out.to_host().astype(np.float64), want, rtol=4e-3, atol=4e-3)
    ai = device.to_device(rng.integers(-5, 5, (8, 16), dtype=np.int8))
    bi = device.to_device(rng.integers(-5, 5, (16, 8), dtype=np.int8))
    with pytest.raises(lib.NoCandidate, match="hipblaslt: .*\n.*ours: .*\n.*host: "):
        lib.matmul(ai, bi)

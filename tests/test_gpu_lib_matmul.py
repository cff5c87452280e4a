"""krn's `lib.matmul` kernel (reference src/krn/lib/lib_kernels.py:31-48) on gfx950, every epilogue of
src/krn/lib/lib_ours.py:38-46: f16 operands run the MFMA GEMM with the bias and activation fused into its epilogue,
f32 operands the generic lowering. Each result is checked against float64 within the float32 accumulation bound
(reference tests/compiler/test_tensor_cores.py:395-401) carried through the activation, plus the output rounding,
and the f32 results against the oracle C backend."""

import math

import numpy as np
import pytest

from krn_amd import T
from oracle import cbackend
from tests.conftest import KERNELS
from tests.kernels import tile_programs as programs
from tests.test_lowering import BASE, EPILOGUES

pytestmark = pytest.mark.gpu

ERF = np.vectorize(math.erf, otypes=[np.float64])
ACT = {
    "relu": lambda x: np.where(x < 0, 0.0, x),
    "gelu": lambda x: 0.5 * x * (1 + ERF(x / math.sqrt(2))),
    "silu": lambda x: x / (1 + np.exp(-x)),
}
# the last two take the skinny kernel (at most 128 rows, K a whole number of 128-byte slices), whose epilogue fetches
# the bias ahead and shares it across lanes; ragged N there
SHAPES = [(50, 38, 70), (256, 512, 256), (130, 257, 64), (100, 130, 64), (7, 45, 192)]


def reference(a, b, bias, flags):
    """float64 result and its bound: the accumulation bound (slope of every activation <= 1.13) plus 8 float32
    ulps for the activation's own arithmetic."""
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    x = a64 @ b64
    err = 8 * 2.0**-24 * (a.shape[1] + 8) * (np.abs(a64) @ np.abs(b64))
    if flags.get("bias"):
        x = x + bias.astype(np.float64)
        err = err + np.abs(x) * 2.0**-24
    for name in ("relu", "gelu", "silu"):
        if flags.get(name):
            x = ACT[name](x)
            err = err * 1.13
    return x, err + np.abs(x) * 8 * 2.0**-24 + 2.0**-126


@pytest.mark.parametrize("name", list(EPILOGUES))
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_f16_lib_matmul_epilogues(device, name, m, n, k):
    flags = EPILOGUES[name]
    rng = np.random.default_rng(11)
    a, b = rng.uniform(-1, 1, (m, k)).astype(np.float16), rng.uniform(-1, 1, (k, n)).astype(np.float16)
    bias = rng.uniform(-2, 2, n).astype(np.float16)
    out = device.empty(T.f16, m, n)
    tiling = programs.MatmulTiling(**flags)
    programs.matmul_epilogue[tiling](device.to_device(a), device.to_device(b), device.to_device(bias), out)
    want, bound = reference(a, b, bias, flags)
    rounded = want.astype(np.float16).astype(np.float64)
    bound = bound + np.abs(rounded - want) + np.spacing(np.abs(rounded).astype(np.float16)).astype(np.float64)
    error = np.abs(out.to_host().astype(np.float64) - want)
    assert np.all(error <= bound), (error - bound).max()


@pytest.mark.parametrize("name", ["bias_gelu", "silu", "bias_relu"])
def test_f32_lib_matmul_matches_the_c_oracle(device, name):
    flags = EPILOGUES[name]
    m, n, k = 70, 90, 40
    rng = np.random.default_rng(12)
    a, b = rng.uniform(-1, 1, (m, k)).astype(np.float32), rng.uniform(-1, 1, (k, n)).astype(np.float32)
    bias = rng.uniform(-2, 2, n).astype(np.float32)
    out = device.empty(T.f32, m, n)
    tiling = programs.MatmulTiling(**flags)
    programs.matmul_epilogue_f32[tiling](device.to_device(a), device.to_device(b), device.to_device(bias), out)
    got = out.to_host()
    want, bound = reference(a, b, bias, flags)
    assert np.all(np.abs(got.astype(np.float64) - want) <= bound)
    # written out in float32 numpy as well, so the check does not rest on the captured program: one fused
    # multiply-add per k in k order, then the bias add and the activation each rounded to float32
    acc = np.zeros((m, n), np.float32)
    for kk in range(k):
        acc = (acc.astype(np.float64) + a[:, kk:kk + 1].astype(np.float64) * b[kk:kk + 1, :]).astype(np.float32)
    if flags.get("bias"):
        acc = acc + bias
    exact = {"relu": lambda x: np.where(x < 0, np.float32(0), x),
             "gelu": lambda x: (np.float32(0.5) * x * (np.float32(1) + ERF(x / np.float32(math.sqrt(2)))
                                                        .astype(np.float32))).astype(np.float32),
             "silu": lambda x: (x / (np.float32(1) + np.exp(-x))).astype(np.float32)}
    for flag, fn in exact.items():
        if flags.get(flag):
            acc = fn(acc)
    np.testing.assert_allclose(got, acc, rtol=8 * 2.0**-23, atol=2.0**-20)
    from krn_amd.compiler.capture import capture

    oracle = np.zeros((m, n), np.float32)
    cbackend.run(capture(KERNELS, "matmul_epilogue_f32", consts={"t": {**BASE, **flags}}), None, [a, b, bias, oracle])
    # same k-ordered fused multiply-adds; erf/exp of the device and host libraries may differ in the last bits
    np.testing.assert_allclose(got, oracle, rtol=4 * 2.0**-23, atol=2.0**-20)

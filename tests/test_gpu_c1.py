"""BASELINE configuration C1 in the GPU run: krn's f32 tile matmul at M=N=K=256, A and B iid U[-1, 1] from a seed.

The reference runs it on its CPU clang backend and checks it against its Python emulator (reference
src/krn/runtime/cpu.py:92-152, src/krn/emulator/emulate.py:305-324). Here the restated pair is checked in this run
(bit-identical, both one fused multiply-add per k in k order), and the same program runs on gfx950 through the generic
lowering, whose f32 product is also one `fmaf` per k in k order: its result is bit-identical to both.
"""

import numpy as np
import pytest

from krn_amd.compiler.capture import capture
from oracle import cbackend, emulate
from tests.conftest import KERNELS
from tests.helpers import assert_agrees
from tests.kernels import tile_programs as programs
from tests.test_oracle import test_c1_f32_gemm_is_bit_identical_between_emulator_and_c_backend_and_within_the_bound

pytestmark = pytest.mark.gpu

TILING = {"bm": 32, "bn": 32, "bk": 16}


def c1_operands():
    rng = np.random.default_rng(0)
    return tuple(rng.uniform(-1, 1, (256, 256)).astype(np.float32) for _ in range(2))


def test_c1_emulator_and_c_backend_agree_bit_for_bit():
    test_c1_f32_gemm_is_bit_identical_between_emulator_and_c_backend_and_within_the_bound()


def test_c1_on_gfx950_is_bit_identical_to_the_emulator_and_the_c_backend(device):
    a, b = c1_operands()
    kernel = capture(KERNELS, "matmul_f32", consts={"t": TILING})
    emulated, compiled = np.zeros((256, 256), np.float32), np.zeros((256, 256), np.float32)
    emulate.run(kernel, None, [a, b, emulated])
    cbackend.run(kernel, None, [a, b, compiled])
    c = device.empty(programs.T.f32, 256, 256)
    launcher = programs.matmul_f32[programs.Tiling(**TILING)]
    explained = launcher.explain(device.to_device(a), device.to_device(b), c)
    assert explained["plan"] == "GenericPlan" and explained["products"] == ["scalar fma"]
    launcher(device.to_device(a), device.to_device(b), c)
    got = c.to_host()
    assert_agrees(got, a, b, 256, "f32")
    np.testing.assert_array_equal(got.view(np.uint32), emulated.view(np.uint32))
    np.testing.assert_array_equal(got.view(np.uint32), compiled.view(np.uint32))

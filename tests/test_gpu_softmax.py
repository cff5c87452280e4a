"""The gfx950 row-softmax kernel (`krn_softmax_rows`), which krn's softmax tile programs lower to (reference
examples/02_tiles_and_types/01_softmax_rows.py:27-40, tests/helpers/example_softmax.py:12-24).

Through the C ABI against a float64 softmax (the function itself: one rounding of the exact value, plus the float32
error of exp and of the running sum) for every element kind, widths around the kernel's register-cache boundary
(4096 columns), the workgroup-per-row form for few long rows (its 16384-column cache) and far past both, odd widths (scalar tails), row strides wider than the row (columns past the width
untouched), and no rows. Through the tile programs against the oracle C backend for bf16 and f32 (f16 is in
test_gpu_generic.py), and that the launch took the kernel, not the generic lowering."""

import numpy as np
import pytest

from krn_amd import Blocks, T
from krn_amd.compiler.capture import capture
from krn_amd.dtypes import BF16, F16, F32, I8
from krn_amd.runtime import library
from oracle import cbackend
from oracle.numerics import bf16_values, bf16_words
from tests.conftest import KERNELS
from tests.kernels import tile_programs as programs

pytestmark = pytest.mark.gpu

# relative tolerance per element kind: half an ulp of the rounding plus float32 exp / sum error
RTOL = {F32: 2e-5, F16: 1.5e-3, BF16: 8e-3}
ATOL = {F32: 1e-30, F16: 3e-8, BF16: 1e-30}  # f16 results below 2^-14 are subnormal: absolute spacing 2^-24
SENTINEL = {F32: np.float32(-7.0), F16: np.float16(-7.0), BF16: np.uint16(0xC0E0)}  # -7.0 in each


def softmax64(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.float64)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def storage(values: np.ndarray, dtype) -> np.ndarray:
    if dtype == BF16:
        return bf16_words(values.astype(np.float32))
    return values.astype(np.float16 if dtype == F16 else np.float32)


def decoded(words: np.ndarray, dtype) -> np.ndarray:
    return bf16_values(words).astype(np.float64) if dtype == BF16 else words.astype(np.float64)


@pytest.mark.parametrize("dtype", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("rows,width,ld", [(1, 1, 1), (5, 7, 7), (3, 4096, 4096), (3, 4097, 4097), (9, 1000, 1024),
                                           (2, 70000, 70000), (130, 512, 520), (11, 8, 8), (0, 64, 64),
                                           (5, 20000, 20008), (4100, 5000, 5000), (4096, 2049, 2049)])
def test_c_abi_softmax_matches_the_float64_softmax(device, dtype, rows, width, ld):
    rng = np.random.default_rng(rows * 100003 + width)
    x = storage(rng.standard_normal((rows, ld)) * 6, dtype)
    y0 = np.full((rows, ld), SENTINEL[dtype])
    dx, dy = device.to_device(x, dtype), device.to_device(y0, dtype)
    library.softmax_rows(dtype, dx.pointer, dy.pointer, rows, width, ld, ld, device.default_stream.handle)
    got = dy.to_host()
    if rows == 0:
        return
    want = softmax64(decoded(x, dtype)[:, :width])
    np.testing.assert_allclose(decoded(got[:, :width], dtype), want, rtol=RTOL[dtype], atol=ATOL[dtype])
    np.testing.assert_array_equal(got[:, width:], y0[:, width:])  # columns past the width untouched
    np.testing.assert_allclose(decoded(got[:, :width], dtype).sum(axis=1), 1.0, rtol=width * RTOL[dtype] + 1e-6)


def test_c_abi_softmax_of_a_row_with_an_infinite_maximum_mass(device):
    """-inf entries take no mass; a row of equal values is uniform; large magnitudes do not overflow."""
    x = np.array([[-np.inf, 0.0, -np.inf, 0.0] * 4, [1e30] * 16, [-1e30, 1e30] * 8], np.float32)
    dx, dy = device.to_device(x), device.empty(T.f32, 3, 16)
    library.softmax_rows(F32, dx.pointer, dy.pointer, 3, 16, 16, 16, device.default_stream.handle)
    got = dy.to_host()
    np.testing.assert_array_equal(got[0], np.array([0.0, 0.125] * 8, np.float32))
    np.testing.assert_array_equal(got[1], np.full(16, 1 / 16, np.float32))
    np.testing.assert_array_equal(got[2], np.array([0.0, 0.125] * 8, np.float32))


def test_c_abi_softmax_refuses_bad_arguments(device):
    dx = device.empty(T.f32, 4, 4)
    with pytest.raises(library.KernelError, match="f32, f16 or bf16"):
        library.softmax_rows(I8, dx.pointer, dx.pointer, 4, 4, 4, 4, device.default_stream.handle)
    with pytest.raises(library.KernelError, match="row strides"):
        library.softmax_rows(F32, dx.pointer, dx.pointer, 4, 8, 4, 4, device.default_stream.handle)


@pytest.mark.parametrize("name,dtype,rows,cols,tile_cols", [
    ("softmax_bf16", BF16, 13, 768, 1024), ("softmax_long_rows_bf16", BF16, 7, 9000, 1024),
    ("softmax_f32", F32, 10, 333, 512), ("softmax_f32", F32, 5, 2048, 1024),
])  # fmt: skip
def test_softmax_programs_take_the_kernel_and_match_the_c_oracle(device, monkeypatch, name, dtype, rows, cols,
                                                                 tile_cols):
    calls = []
    real = library.softmax_rows
    monkeypatch.setattr(library, "softmax_rows", lambda *a: (calls.append(a), real(*a)))
    rng = np.random.default_rng(rows * cols)
    x = storage(rng.standard_normal((rows, cols)) * 4, dtype)
    tiling = programs.RowTiling(rows=4, cols=tile_cols)
    y = device.empty(T.bf16 if dtype == BF16 else T.f32, rows, cols)
    launch = Blocks(-(-rows // 4))
    if name.startswith("softmax_long_rows"):
        getattr(programs, name)(tiling, device.to_device(x, dtype), y, launch=launch)
    else:
        getattr(programs, name)(device.to_device(x, dtype), y, tiling, launch=launch)
    assert len(calls) == 1 and calls[0][3] == rows
    kernel = capture(KERNELS, name, consts={"t": {"rows": 4, "cols": tile_cols}})
    want = np.zeros((rows, cols), x.dtype)
    cbackend.run(kernel, launch, [x, want])
    got = y.to_host()
    width = cols if name.startswith("softmax_long_rows") else min(cols, tile_cols)
    assert calls[0][4] == width
    np.testing.assert_allclose(decoded(got[:, :width], dtype), decoded(want[:, :width], dtype), rtol=RTOL[dtype],
                               atol=ATOL[dtype])


@pytest.mark.parametrize("name,config,rows,cols", [("running", "Rows", 10, 3000), ("one_tile", "Tile", 37, 96)])
def test_rewritten_softmax_programs_take_the_kernel(device, name, config, rows, cols):
    """krn's row softmax spelled another way (names, operand order, temporaries): planned as the row-softmax kernel
    and equal to a float64 softmax of the valid columns."""
    from tests.kernels import softmax_variants as variants

    rng = np.random.default_rng(11)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float16)
    y = device.empty(T.f16, rows, cols)
    cfg = getattr(variants, config)()
    launcher = device.launcher(getattr(variants, name), Blocks(-(-rows // cfg.per_block)))
    assert launcher.explain(cfg, device.to_device(x), y)["plan"] == "SoftmaxPlan"
    launcher(cfg, device.to_device(x), y)
    np.testing.assert_allclose(y.to_host().astype(np.float64), softmax64(x), rtol=RTOL[F16], atol=ATOL[F16])

"""Tile programs outside the MFMA kernels run through the generic hiprtc lowering and match the oracle C backend:
transposes, where, comparisons, arange positions, bare products, per-head slices, causal masks, reductions
(reference tests/frontend/test_tile_ops.py:54-118)."""

import math

import numpy as np
import pytest

from krn_amd import Blocks, T
from krn_amd.compiler.capture import capture
from oracle import cbackend, emulate
from tests.conftest import KERNELS
from tests.kernels import tile_programs as programs

pytestmark = pytest.mark.gpu

SIZES = [(1, 1), (5, 11), (8, 16), (3, 16), (8, 2)]


def on_gpu(device, name, arrays, launch=Blocks(1), dtypes=None):
    tensors = [device.to_device(a) for a in arrays]
    getattr(programs, name)(programs.Shape(), *tensors, launch=launch)
    return [t.to_host() for t in tensors]


def on_oracle(name, arrays, launch=Blocks(1)):
    kernel = capture(KERNELS, name)
    copies = [a.copy() for a in arrays]
    cbackend.run(kernel, launch, copies)
    return copies


@pytest.mark.parametrize("size", SIZES)
@pytest.mark.parametrize("name", ["transpose", "select", "causal", "scaled_by_extent", "row_softmax"])
def test_elementwise_tile_programs_match_the_c_oracle(device, name, size):
    rng = np.random.default_rng(sum(size))
    x = rng.standard_normal(size).astype(np.float32)
    out = np.full(size[::-1] if name == "transpose" else size, -7.0, np.float32)
    got = on_gpu(device, name, [x, out])
    want = on_oracle(name, [x, out])
    if name == "row_softmax":  # expf differs between the GPU and glibc by an ulp or two
        np.testing.assert_allclose(got[1], want[1], rtol=2e-6, atol=1e-7)
    else:
        np.testing.assert_array_equal(got[1], want[1])


@pytest.mark.parametrize("size", SIZES)
def test_elementwise_tile_programs_match_numpy(device, size):
    """The same programs against expectations written out in numpy (reference tests/frontend/test_tile_ops.py:54-118,
    212-213), so a capture mistake shared by the device path and the oracle cannot pass: rows and columns past the
    tensor's edge are invalid lanes and are neither read nor stored."""
    rng = np.random.default_rng(100 + sum(size))
    x = rng.standard_normal(size).astype(np.float32)
    keep = np.arange(size[1])[None, :] <= np.arange(size[0])[:, None]
    expected = {
        "transpose": x.T,
        "select": np.where(x > 0, x, np.float32(0.5)),
        "causal": np.where(keep, x, np.float32(-1.0e30)),
        "scaled_by_extent": x * np.float32(programs.Shape().cols),  # the tile's extent, not the valid width
    }
    for name, want in expected.items():
        out = np.full(want.shape, -7.0, np.float32)
        np.testing.assert_array_equal(on_gpu(device, name, [x, out])[1], want, err_msg=name)


@pytest.mark.parametrize("size", SIZES)
def test_comparisons_and_positions_are_exact(device, size):
    rng = np.random.default_rng(5)
    x = np.round(rng.standard_normal(size)).astype(np.float32)
    outs = [np.zeros(size, np.float32) for _ in range(4)]
    got = on_gpu(device, "compare", [x, *outs])
    for g, want in zip(got[1:], [(x < 0), (x <= 0), (x > 0), (x >= 0)]):
        np.testing.assert_array_equal(g, want.astype(np.float32))
    positions = on_gpu(device, "positions", [np.zeros(size, np.int32)])[0]
    np.testing.assert_array_equal(positions, np.arange(size[1])[None, :] - (np.arange(size[0])[:, None] + 3))


@pytest.mark.parametrize("size", SIZES)
def test_bare_product_and_per_head_match_the_oracle(device, size):
    rng = np.random.default_rng(6)
    x, w = rng.standard_normal(size).astype(np.float16), rng.standard_normal((8, size[1])).astype(np.float16)
    y = np.zeros((8, 8), np.float32)
    got = on_gpu(device, "product", [x, w, y])[2]
    want = on_oracle("product", [x, w, y])[2]
    np.testing.assert_array_equal(got, want)  # same k-ordered fused multiply-adds on both
    heads = 3
    x3 = rng.standard_normal((heads, *size)).astype(np.float32)
    got = on_gpu(device, "per_head", [x3, np.zeros_like(x3)], Blocks(1, heads))[1]
    np.testing.assert_array_equal(got, 2 * x3)


def test_flash_attention_with_a_small_head_dimension_runs_generic_and_matches_the_emulator(device):
    """d = 16 is not a head dimension of the MFMA attention kernel, so the generic lowering runs it."""
    rng = np.random.default_rng(7)
    heads, seq, d = 2, 37, 16
    q, k, v = (rng.standard_normal((heads, seq, d)).astype(np.float16) for _ in range(3))
    consts = {"bq": 8, "bk": 8, "d": d, "causal": True}
    scale = math.log2(math.e) / math.sqrt(d)
    launch = Blocks(-(-seq // 8), heads)
    o = device.empty(T.f16, heads, seq, d)
    programs.flash_attention(programs.Attention(**consts), *(device.to_device(x) for x in (q, k, v)), o, scale,
                             launch=launch)
    want = np.zeros((heads, seq, d), np.float16)
    emulate.run(capture(KERNELS, "flash_attention", consts={"t": consts}), launch, [q, k, v, want, scale])
    np.testing.assert_allclose(o.to_host().astype(np.float32), want.astype(np.float32), atol=1e-3)


@pytest.mark.parametrize("path", ["kernel", "generic"])
@pytest.mark.parametrize("name,rows,cols,tile_cols", [("softmax_long_rows", 6, 2500, 1024),
                                                      ("softmax_long_rows", 37, 5000, 1024), ("softmax", 6, 512, 512),
                                                      ("softmax_steps", 9, 4096, 4096), ("softmax", 10, 700, 512)])
def test_softmax_programs_match_the_c_oracle(device, name, rows, cols, tile_cols, path):
    """krn's softmax programs (reference examples/02_tiles_and_types/01_softmax_rows.py, the long rows in ragged
    column chunks; tests/helpers/example_softmax.py) against the oracle C backend: the same f32 arithmetic, so f16
    results within an ulp (exp differs between the GPU and glibc in the last bits). One block per 4 rows takes the
    row-softmax kernel; one block more keeps the program's own meaning on the generic lowering."""
    rng = np.random.default_rng(rows * cols)
    x = (rng.standard_normal((rows, cols)) * 4).astype(np.float16)
    tiling = programs.RowTiling(rows=4, cols=tile_cols)
    y = device.empty(T.f16, rows, cols)
    y.copy_from(np.zeros((rows, cols), np.float16))
    launch = Blocks(-(-rows // 4) + (path == "generic"))
    if name == "softmax_long_rows":
        programs.softmax_long_rows(tiling, device.to_device(x), y, launch=launch)
    else:
        getattr(programs, name)(device.to_device(x), y, tiling, launch=launch)
    kernel = capture(KERNELS, name, consts={"t": {"rows": 4, "cols": tile_cols}})
    want = np.zeros((rows, cols), np.float16)
    cbackend.run(kernel, launch, [x, want])
    np.testing.assert_allclose(y.to_host().astype(np.float32), want.astype(np.float32), rtol=2e-3, atol=2e-6)

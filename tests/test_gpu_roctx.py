"""Tile program launches inside ROCTx ranges (`launch_ranges(True)`) on gfx950: the same results as without."""

import numpy as np
import pytest

from krn_amd import Blocks, T
from krn_amd.hw import Libraries
from krn_amd.runtime import roctx
from tests.kernels import tile_programs as programs

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(Libraries.find("roctx") is None, reason="no ROCTx library on this machine")]


def test_launches_in_ranges_give_the_same_results(device):
    rng = np.random.default_rng(41)
    x = device.to_device((rng.standard_normal((37, 900)) * 3).astype(np.float16))
    y = device.empty(T.f16, 37, 900)
    tiling = programs.RowTiling(rows=4, cols=1024)
    programs.softmax(x, y, tiling, launch=Blocks(10))
    want = y.to_host()
    before = roctx.launch_ranges()
    try:
        roctx.launch_ranges(True)
        y.copy_from(np.zeros((37, 900), np.float16))
        with roctx.span("krn_amd test"):
            programs.softmax(x, y, tiling, launch=Blocks(10))
        np.testing.assert_array_equal(y.to_host(), want)
    finally:
        roctx.launch_ranges(before)

"""The four-wave whole-tile GEMM loop (gemm_quad16) at every K length its six-slice unrolled loop treats
differently: the loop runs whole groups of six 128-byte K slices and then a tail of one to five, the first two
slices come from the prologue, and the loads of the last two slices re-read the last one. Each product here has at
least 128 tiles of 256 x 256 (so the dispatch picks this loop), a ragged last row of tiles (M = 2008), and is
checked on sampled rows: bf16 and fp8 against the float64 product within the accumulation bound plus the bf16
output rounding, int8 bit-exact against the integer product, and the NN form (B read K x N as it lies) bit-identical
to the NT product on the transposed operand."""

import numpy as np
import pytest

from krn_amd import T
from krn_amd.dtypes import BF16, F8E4M3, I8, I32
from krn_amd.runtime import library
from oracle.numerics import bf16_values, e4m3_decode, e4m3_encode
from tests.helpers import assert_agrees, bf16_normal

pytestmark = pytest.mark.gpu

M, N = 2008, 4096  # 8 x 16 = 128 tiles, the last row of tiles 216 rows high
SLICES = [2, 3, 4, 5, 6, 7, 8, 13]
ROWS = np.array([0, 1, 127, 255, 256, 1023, 1792, 2000, M - 1])


@pytest.mark.parametrize("slices", SLICES)
def test_bf16_every_tail_length(device, slices):
    k = 64 * slices
    rng = np.random.default_rng(slices)
    aw, av = bf16_normal(rng, (M, k))
    bw, bv = bf16_normal(rng, (N, k))
    c = device.empty(T.bf16, M, N)
    a, b = device.to_device(aw, T.bf16), device.to_device(bw, T.bf16)
    library.gemm_nt(BF16, a.pointer, b.pointer, c.pointer, BF16, M, N, k, [], device.default_stream.handle)
    got = bf16_values(c.to_host()[ROWS])
    assert_agrees(got, av[ROWS], bv.T, k, "bf16")


@pytest.mark.parametrize("slices", SLICES)
def test_fp8_every_tail_length(device, slices):
    k = 128 * slices
    rng = np.random.default_rng(100 + slices)
    ac = e4m3_encode(rng.standard_normal((M, k)).astype(np.float32))
    bc = e4m3_encode(rng.standard_normal((N, k)).astype(np.float32))
    c = device.empty(T.bf16, M, N)
    a, b = device.to_device(ac, T.f8e4m3fn), device.to_device(bc, T.f8e4m3fn)
    library.gemm_nt(F8E4M3, a.pointer, b.pointer, c.pointer, BF16, M, N, k, [], device.default_stream.handle)
    got = bf16_values(c.to_host()[ROWS])
    assert_agrees(got, e4m3_decode(ac[ROWS]), e4m3_decode(bc).T, k, "bf16")


@pytest.mark.parametrize("slices", SLICES)
def test_int8_every_tail_length_is_exact(device, slices):
    k = 128 * slices
    rng = np.random.default_rng(200 + slices)
    ah = rng.integers(-128, 128, (M, k), dtype=np.int8)
    bh = rng.integers(-128, 128, (N, k), dtype=np.int8)
    c = device.empty(T.i32, M, N)
    a, b = device.to_device(ah, T.i8), device.to_device(bh, T.i8)
    library.gemm_nt(I8, a.pointer, b.pointer, c.pointer, I32, M, N, k, [], device.default_stream.handle)
    want = ah[ROWS].astype(np.int64) @ bh.astype(np.int64).T
    np.testing.assert_array_equal(c.to_host()[ROWS].astype(np.int64), want)


@pytest.mark.parametrize("slices", [2, 3, 5, 7, 13])
def test_bf16_nn_every_tail_length_equals_nt(device, slices):
    k = 64 * slices
    rng = np.random.default_rng(300 + slices)
    aw, _ = bf16_normal(rng, (M, k))
    bw, _ = bf16_normal(rng, (k, N))
    a, b = device.to_device(aw, T.bf16), device.to_device(bw, T.bf16)
    bt = device.to_device(np.ascontiguousarray(bw.T), T.bf16)
    c_nn, c_nt = device.empty(T.bf16, M, N), device.empty(T.bf16, M, N)
    stream = device.default_stream.handle
    library.check(library.lib().krn_gemm_nn(library.kind(BF16), a.pointer, b.pointer, c_nn.pointer,
                                            library.kind(BF16), M, N, k, 0, None, None, None, None, 0, stream),
                  "krn_gemm_nn")
    library.gemm_nt(BF16, a.pointer, bt.pointer, c_nt.pointer, BF16, M, N, k, [], stream)
    np.testing.assert_array_equal(c_nn.to_host(), c_nt.to_host())

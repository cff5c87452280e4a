"""The tile GEMM programs on gfx950 against krn's oracles: the forward-error bound of float64 numpy (krn's `agree`),
the oracle emulator and C backend on the same seeded inputs, and exact integer arithmetic for int8."""

import numpy as np
import pytest

from krn_amd import T
from oracle import cbackend, emulate
from oracle.numerics import bf16_values, bf16_words, e4m3_decode, e4m3_encode
from tests.conftest import KERNELS
from tests.helpers import assert_agrees, bf16_normal
from tests.kernels import tile_programs as programs

pytestmark = pytest.mark.gpu

SHAPES = [(50, 38, 72), (257, 129, 40), (512, 512, 512), (300, 1000, 136), (50, 38, 70), (16, 8, 8), (130, 257, 33),
          (1, 384, 256), (16, 8, 0), (40, 300, 128), (70, 96, 384), (97, 33, 64)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_bf16_nt_gemm_agrees_with_the_float64_bound(device, m, n, k):
    rng = np.random.default_rng(0)
    (aw, a), (bw, b) = bf16_normal(rng, (m, k)), bf16_normal(rng, (n, k))
    c = device.empty(T.bf16, m, n)
    programs.gemm_nt[programs.Tiling(bm=64, bn=64, bk=32)](device.to_device(aw, T.bf16), device.to_device(bw, T.bf16), c)
    got = bf16_values(c.to_host())
    assert_agrees(got, a, b.T, k, "bf16")


@pytest.mark.parametrize("m,n,k", SHAPES[:6])
def test_bf16_gemm_with_f32_output_is_within_the_bound_and_close_to_the_c_oracle(device, m, n, k):
    rng = np.random.default_rng(1)
    (aw, a), (bw, b) = bf16_normal(rng, (m, k)), bf16_normal(rng, (n, k))
    c = device.empty(T.f32, m, n)
    tiling = programs.Tiling(bm=32, bn=32, bk=16)
    programs.gemm_nt_f32[tiling](device.to_device(aw, T.bf16), device.to_device(bw, T.bf16), c)
    got = c.to_host()
    assert_agrees(got, a, b.T, k, "f32")
    from krn_amd.compiler.capture import capture

    oracle = np.zeros((m, n), np.float32)
    kernel = capture(KERNELS, "gemm_nt_f32", consts={"t": {"bm": 32, "bn": 32, "bk": 16}})
    cbackend.run(kernel, None, [aw, bw, oracle])
    assert_agrees(oracle, a, b.T, k, "f32")


@pytest.mark.parametrize("m,n,k", [(50, 38, 70), (130, 257, 64), (512, 256, 384)])
def test_f16_nn_matmul_example_agrees(device, m, n, k):
    """krn's own GEMM example program (b is K x N) with an f16 result."""
    rng = np.random.default_rng(2)
    a, b = rng.uniform(-1, 1, (m, k)).astype(np.float16), rng.uniform(-1, 1, (k, n)).astype(np.float16)
    c = device.empty(T.f16, m, n)
    programs.matmul[programs.Tiling(bm=16, bn=16, bk=8)](device.to_device(a), device.to_device(b), c)
    assert_agrees(c.to_host(), a.astype(np.float32), b.astype(np.float32), k, "f16")


def fp8_operands(rng, m, n, k):
    x, w = rng.standard_normal((m, k)).astype(np.float32), rng.standard_normal((n, k)).astype(np.float32)
    sx, sw = np.float32(np.abs(x).max() / 448), np.float32(np.abs(w).max() / 448)
    return e4m3_encode(x / sx), e4m3_encode(w / sw), sx, sw


@pytest.mark.parametrize("m,n,k", [(1, 256, 512), (16, 384, 256), (128, 640, 1024), (200, 130, 96), (50, 38, 72)])
def test_fp8_gemm_with_per_tensor_scales(device, m, n, k):
    rng = np.random.default_rng(81)
    a, b, sa, sb = fp8_operands(rng, m, n, k)
    c = device.empty(T.bf16, m, n)
    programs.gemm_fp8[programs.Tiling(bm=64, bn=64, bk=64)](
        device.to_device(a, T.f8e4m3fn), device.to_device(b, T.f8e4m3fn), c, sa, sb)
    got = bf16_values(c.to_host()).astype(np.float64)
    da, db = e4m3_decode(a).astype(np.float64), e4m3_decode(b).astype(np.float64)
    scale = np.float64(np.float32(sa * sb))
    reference = (da @ db.T) * scale
    bound = (8 * 2.0**-24 * (k + 8) * (np.abs(da) @ np.abs(db).T)) * scale + np.abs(reference) * 2.0**-8 * 1.01
    assert np.all(np.abs(got - reference) <= bound + 1e-30)


def test_fp8_gemm_matches_the_oracle_emulator(device):
    rng = np.random.default_rng(82)
    m, n, k = 40, 72, 128
    a, b, sa, sb = fp8_operands(rng, m, n, k)
    c = device.empty(T.bf16, m, n)
    programs.gemm_fp8[programs.Tiling(bm=32, bn=32, bk=32)](
        device.to_device(a, T.f8e4m3fn), device.to_device(b, T.f8e4m3fn), c, sa, sb)
    from krn_amd.compiler.capture import capture

    kernel = capture(KERNELS, "gemm_fp8", consts={"t": {"bm": 32, "bn": 32, "bk": 32}})
    want = np.zeros((m, n), np.uint16)
    emulate.run(kernel, None, [a, b, want, sa, sb])
    got, expected = bf16_values(c.to_host()).astype(np.float64), bf16_values(want).astype(np.float64)
    # accumulation order differs (MFMA vs k-ordered FMA): both are within the float32 bound of the exact product,
    # so they differ by at most twice that bound plus one bf16 rounding each
    da, db = e4m3_decode(a).astype(np.float64), e4m3_decode(b).astype(np.float64)
    scale = np.float64(np.float32(sa * sb))
    accumulation = 8 * 2.0**-24 * (k + 8) * (np.abs(da) @ np.abs(db).T) * scale
    assert np.all(np.abs(got - expected) <= 2 * accumulation + (np.abs(got) + np.abs(expected)) * 2.0**-8)


@pytest.mark.parametrize("m,n,k", [(16, 640, 512), (100, 300, 256), (257, 129, 96), (5, 7, 3)])
def test_int8_gemm_int32_is_bit_exact(device, m, n, k):
    rng = np.random.default_rng(3)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    c = device.empty(T.i32, m, n)
    programs.gemm_i8_i32[programs.Tiling(bm=32, bn=32, bk=32)](device.to_device(a), device.to_device(w), c)
    np.testing.assert_array_equal(c.to_host(), a.astype(np.int64) @ w.astype(np.int64).T)


# 33..128 rows with K a whole number of 128-byte slices take the LDS-staged skinny kernel: fewer slices than waves
# (k=128: one), remainders (3, 5, 7, 9 slices over four waves), ragged rows and columns
@pytest.mark.parametrize("m,n,k", [(33, 96, 128), (64, 64, 384), (65, 130, 1152), (96, 33, 640), (127, 100, 896),
                                   (128, 256, 2048)])
def test_int8_skinny_staged_is_bit_exact(device, m, n, k):
    rng = np.random.default_rng(5)
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    w = rng.integers(-128, 128, (n, k), dtype=np.int8)
    c = device.empty(T.i32, m, n)
    programs.gemm_i8_i32[programs.Tiling(bm=32, bn=32, bk=32)](device.to_device(a), device.to_device(w), c)
    np.testing.assert_array_equal(c.to_host(), a.astype(np.int64) @ w.astype(np.int64).T)


# one row block (M <= 32): only the eight-row groups of A holding rows < M are loaded (1 to 4 of them); the ring rows
# past them hold stale LDS contents whose results are never stored. Every group boundary, with slice counts below,
# at and above the four-stage ring per wave.
@pytest.mark.parametrize("m", [1, 7, 8, 9, 16, 17, 24, 25, 32])
@pytest.mark.parametrize("k", [128, 1024, 128 * 37])
def test_int8_single_row_block_loads_only_the_rows_it_needs(device, m, k):
    rng = np.random.default_rng(m * 1000 + k)
    n = 200
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    w = rng.integers(-128, 128, (n, k), dtype=np.int8)
    c = device.empty(T.i32, m, n)
    programs.gemm_i8_i32[programs.Tiling(bm=32, bn=32, bk=32)](device.to_device(a), device.to_device(w), c)
    np.testing.assert_array_equal(c.to_host(), a.astype(np.int64) @ w.astype(np.int64).T)


@pytest.mark.parametrize("m,n,k", [(33, 96, 64), (100, 70, 320), (128, 256, 1088)])
def test_bf16_skinny_staged_agrees_with_the_float64_bound(device, m, n, k):
    rng = np.random.default_rng(6)
    (aw, a), (bw, b) = bf16_normal(rng, (m, k)), bf16_normal(rng, (n, k))
    c = device.empty(T.bf16, m, n)
    programs.gemm_nt[programs.Tiling(bm=64, bn=64, bk=32)](device.to_device(aw, T.bf16), device.to_device(bw, T.bf16), c)
    assert_agrees(bf16_values(c.to_host()), a, b.T, k, "bf16")


# At least 256 tiles of 256 x 256 with ragged M and N take the pipelined whole-tile kernels: the rows past the end of
# A and B load zeros through the buffer resources' bounds and the epilogue stores only the inside
RAGGED = [(4000, 4100, 256), (4097, 3969, 128), (3841, 4351, 384)]


# Up to 256 tiles of 128 x 128 (and more than 128 rows) take the pipelined loop on 128 x 128 tiles
MID = [(1000, 1100, 256), (512, 2048, 384), (1500, 2000, 128)]
# more than 256 tiles of 128 x 128 but fewer than 128 of 256 x 256: 128 x 256 tiles (fp8: the staged tiles); and
# from 128 tiles of 256 x 256 on, the 256 x 256 loop with ragged edges
BAND = [(2560, 2600, 256), (2400, 2900, 128), (3000, 3100, 256)]


@pytest.mark.parametrize("m,n,k", BAND)
def test_bf16_band_sizes_agree_with_the_float64_bound(device, m, n, k):
    rng = np.random.default_rng(13)
    (aw, a), (bw, b) = bf16_normal(rng, (m, k)), bf16_normal(rng, (n, k))
    c = device.empty(T.bf16, m, n)
    programs.gemm_nt[programs.Tiling(bm=64, bn=64, bk=32)](device.to_device(aw, T.bf16), device.to_device(bw, T.bf16), c)
    assert_agrees(bf16_values(c.to_host()), a, b.T, k, "bf16")


@pytest.mark.parametrize("m,n,k", BAND)
def test_int8_band_sizes_are_bit_exact(device, m, n, k):
    rng = np.random.default_rng(14)
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    w = rng.integers(-128, 128, (n, k), dtype=np.int8)
    c = device.empty(T.i32, m, n)
    programs.gemm_i8_i32[programs.Tiling(bm=32, bn=32, bk=32)](device.to_device(a), device.to_device(w), c)
    np.testing.assert_array_equal(c.to_host(), (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.int64))


@pytest.mark.parametrize("m,n,k", MID)
def test_bf16_mid_size_agrees_with_the_float64_bound(device, m, n, k):
    rng = np.random.default_rng(10)
    (aw, a), (bw, b) = bf16_normal(rng, (m, k)), bf16_normal(rng, (n, k))
    c = device.empty(T.bf16, m, n)
    programs.gemm_nt[programs.Tiling(bm=64, bn=64, bk=32)](device.to_device(aw, T.bf16), device.to_device(bw, T.bf16), c)
    assert_agrees(bf16_values(c.to_host()), a, b.T, k, "bf16")


@pytest.mark.parametrize("m,n,k", MID)
def test_int8_mid_size_is_bit_exact(device, m, n, k):
    rng = np.random.default_rng(11)
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    w = rng.integers(-128, 128, (n, k), dtype=np.int8)
    c = device.empty(T.i32, m, n)
    programs.gemm_i8_i32[programs.Tiling(bm=32, bn=32, bk=32)](device.to_device(a), device.to_device(w), c)
    np.testing.assert_array_equal(c.to_host(), (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.int64))


@pytest.mark.parametrize("m,n,k", MID[:2])
def test_fp8_mid_size_with_per_tensor_scales(device, m, n, k):
    rng = np.random.default_rng(12)
    a, b, sa, sb = fp8_operands(rng, m, n, k)
    c = device.empty(T.bf16, m, n)
    programs.gemm_fp8[programs.Tiling(bm=64, bn=64, bk=64)](
        device.to_device(a, T.f8e4m3fn), device.to_device(b, T.f8e4m3fn), c, sa, sb)
    got = bf16_values(c.to_host()).astype(np.float64)
    da, db = e4m3_decode(a).astype(np.float64), e4m3_decode(b).astype(np.float64)
    scale = np.float64(np.float32(sa * sb))
    reference = (da @ db.T) * scale
    bound = (8 * 2.0**-24 * (k + 8) * (np.abs(da) @ np.abs(db).T)) * scale + np.abs(reference) * 2.0**-8 * 1.01
    assert np.all(np.abs(got - reference) <= bound + 1e-30)


@pytest.mark.parametrize("m,n,k", RAGGED)
def test_bf16_ragged_whole_tiles_agree_with_the_float64_bound(device, m, n, k):
    rng = np.random.default_rng(7)
    (aw, a), (bw, b) = bf16_normal(rng, (m, k)), bf16_normal(rng, (n, k))
    c = device.empty(T.bf16, m, n)
    programs.gemm_nt[programs.Tiling(bm=64, bn=64, bk=32)](device.to_device(aw, T.bf16), device.to_device(bw, T.bf16), c)
    assert_agrees(bf16_values(c.to_host()), a, b.T, k, "bf16")


@pytest.mark.parametrize("m,n,k", RAGGED)
def test_w8a8_ragged_whole_tiles_are_bit_exact(device, m, n, k):
    """int32 accumulation is exact (float64 holds it), so the result is bf16(f32(f32(acc) * sa[m]) * sw[n])."""
    rng = np.random.default_rng(8)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    sa = (rng.uniform(0.5, 1.5, (m, 1)) / 127).astype(np.float32)
    sw = (rng.uniform(0.5, 1.5, (1, n)) / 127).astype(np.float32)
    c = device.empty(T.bf16, m, n)
    programs.gemm_w8a8[programs.Tiling(bm=32, bn=32, bk=32)](device.to_device(a), device.to_device(w),
                                                           device.to_device(sa), device.to_device(sw), c)
    acc = (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)
    want = bf16_words((acc * sa).astype(np.float32) * sw)
    np.testing.assert_array_equal(c.to_host(), want)


@pytest.mark.parametrize("m,n,k", RAGGED[:2])
def test_fp8_ragged_whole_tiles_with_per_tensor_scales(device, m, n, k):
    rng = np.random.default_rng(9)
    a, b, sa, sb = fp8_operands(rng, m, n, k)
    c = device.empty(T.bf16, m, n)
    programs.gemm_fp8[programs.Tiling(bm=64, bn=64, bk=64)](
        device.to_device(a, T.f8e4m3fn), device.to_device(b, T.f8e4m3fn), c, sa, sb)
    got = bf16_values(c.to_host()).astype(np.float64)
    da, db = e4m3_decode(a).astype(np.float64), e4m3_decode(b).astype(np.float64)
    scale = np.float64(np.float32(sa * sb))
    reference = (da @ db.T) * scale
    bound = (8 * 2.0**-24 * (k + 8) * (np.abs(da) @ np.abs(db).T)) * scale + np.abs(reference) * 2.0**-8 * 1.01
    assert np.all(np.abs(got - reference) <= bound + 1e-30)


@pytest.mark.parametrize("m,n,k", [(16, 512, 256), (96, 200, 160), (33, 65, 64), (33, 65, 128), (100, 70, 384),
                                   (128, 200, 256)])
def test_w8a8_dequant_epilogue_is_bit_exact_against_the_oracle(device, m, n, k):
    """int32 accumulation is exact, so the whole result is: bf16(f32(f32(acc) * sa[m]) * sw[n])."""
    rng = np.random.default_rng(4)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    sa = (rng.uniform(0.5, 1.5, (m, 1)) / 127).astype(np.float32)
    sw = (rng.uniform(0.5, 1.5, (1, n)) / 127).astype(np.float32)
    c = device.empty(T.bf16, m, n)
    tiling = programs.Tiling(bm=32, bn=32, bk=32)
    programs.gemm_w8a8[tiling](device.to_device(a), device.to_device(w), device.to_device(sa), device.to_device(sw), c)
    from krn_amd.compiler.capture import capture

    kernel = capture(KERNELS, "gemm_w8a8", consts={"t": {"bm": 32, "bn": 32, "bk": 32}})
    want = np.zeros((m, n), np.uint16)
    emulate.run(kernel, None, [a, w, sa, sw, want])
    np.testing.assert_array_equal(c.to_host(), want)

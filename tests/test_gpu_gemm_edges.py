"""Edges of the tile GEMM on gfx950: empty outputs, special values and the full int8 range.

The reference's products are IEEE arithmetic (its CPU backend is one `fmaf` per k, reference
src/krn/compiler/emit.py:791-796), so a NaN operand makes its whole output row or column NaN, an infinity makes it
infinite, and infinity times zero is NaN. Each shape below is chosen to reach one of the kernel families (the
mid-size and whole-tile pipelines, the skinny kernel and the bounds-checked tiles), because each has its own
epilogue store."""

import numpy as np
import pytest

from krn_amd import T
from krn_amd.dtypes import BF16, F16, F32, I8
from krn_amd.runtime import hipapi, library
from oracle.numerics import bf16_values, bf16_words, e4m3_decode, e4m3_encode
from tests.helpers import agree_bound, assert_agrees
from tests.kernels import tile_programs as programs

pytestmark = pytest.mark.gpu

TILING = programs.Tiling(bm=64, bn=64, bk=32)


@pytest.mark.parametrize("m,n,k", [(0, 64, 128), (64, 0, 128), (0, 0, 0)])
def test_an_empty_output_launches_nothing_and_raises_nothing(device, m, n, k):
    a = device.to_device(np.zeros((m, k), np.uint16), T.bf16)
    b = device.to_device(np.zeros((n, k), np.uint16), T.bf16)
    c = device.empty(T.bf16, m, n)
    programs.gemm_nt[TILING](a, b, c)
    device.default_stream.sync()
    assert c.to_host().shape == (m, n)


def classes(x: np.ndarray) -> np.ndarray:
    """0 finite, 1 NaN, 2 +inf, 3 -inf."""
    return np.select([np.isnan(x), x == np.inf, x == -np.inf], [1, 2, 3], 0)


# (m, n, k): mid-size pipeline, whole 256 x 256 pipeline, skinny, bounds-checked tiles (K not whole 128-byte slices)
SPECIAL_SHAPES = [(512, 512, 256), (2048, 4096, 128), (16, 640, 512), (300, 200, 136)]


@pytest.mark.parametrize("m,n,k", SPECIAL_SHAPES)
def test_bf16_special_values_propagate_as_in_ieee_arithmetic(device, m, n, k):
    rng = np.random.default_rng(m + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k)).astype(np.float32)
    a[3, 5] = np.nan          # row 3: NaN
    a[7, 9] = np.inf          # row 7: +-inf, and NaN in the columns whose B row is 0 at k = 9
    b[11, 9] = 0.0
    b[13, 2] = -np.inf        # column 13: +-inf, NaN where A's row meets it with 0 or with the +inf above
    a[8, 2] = 0.0
    aw, bw = bf16_words(a), bf16_words(b)
    av, bv = bf16_values(aw).astype(np.float64), bf16_values(bw).astype(np.float64)
    c = device.empty(T.bf16, m, n)
    programs.gemm_nt[TILING](device.to_device(aw, T.bf16), device.to_device(bw, T.bf16), c)
    got = bf16_values(c.to_host()).astype(np.float64)
    with np.errstate(invalid="ignore"):
        want = np.einsum("ik,jk->ij", av, bv)
    np.testing.assert_array_equal(classes(got), classes(want))
    assert np.isnan(got[3]).all() and np.isnan(got[8, 13]) and np.isnan(got[7, 11])
    # a finite entry's A row and B row hold no special value, so it is the product of the operands with the
    # special values zeroed: krn's float32 bound plus one bf16 rounding there
    finite = classes(want) == 0
    clean_a, clean_b = np.where(np.isfinite(av), av, 0.0), np.where(np.isfinite(bv), bv, 0.0)
    reference, bound = agree_bound(clean_a, clean_b.T, k)
    bound = bound + np.abs(reference) * 2.0**-8 + 2.0**-133
    assert np.all(np.abs(got - reference)[finite] <= bound[finite])


@pytest.mark.parametrize("m,n,k", [(512, 512, 256), (16, 640, 512), (100, 200, 200)])
def test_fp8_nan_codes_make_their_row_and_column_nan(device, m, n, k):
    """e4m3fn has no infinity; 0x7F and 0xFF are NaN (reference narrow.py:94-110). A NaN code in A poisons its row,
    one in B its column, through the scale epilogue as well."""
    rng = np.random.default_rng(7)
    a = e4m3_encode(rng.standard_normal((m, k)).astype(np.float32))
    b = e4m3_encode(rng.standard_normal((n, k)).astype(np.float32))
    a[2, 17], b[5, 40] = 0x7F, 0xFF
    c = device.empty(T.bf16, m, n)
    programs.gemm_fp8[TILING](device.to_device(a, T.f8e4m3fn), device.to_device(b, T.f8e4m3fn), c, 0.5, 0.25)
    got = bf16_values(c.to_host()).astype(np.float64)
    want_nan = np.zeros((m, n), bool)
    want_nan[2, :] = True
    want_nan[:, 5] = True
    np.testing.assert_array_equal(np.isnan(got), want_nan)
    da, db = e4m3_decode(a).astype(np.float64), e4m3_decode(b).astype(np.float64)
    da[2], db[5] = 0.0, 0.0
    keep = ~want_nan
    scale = 0.5 * 0.25
    reference = (da @ db.T) * scale
    bound = (8 * 2.0**-24 * (k + 8) * (np.abs(da) @ np.abs(db).T)) * scale + np.abs(reference) * 2.0**-8 * 1.01
    assert np.all(np.abs(got - reference)[keep] <= bound[keep] + 1e-30)


@pytest.mark.parametrize("m,n,k", [(512, 768, 384), (16, 640, 512), (257, 129, 96)])
def test_int8_gemm_over_the_full_int8_range_is_bit_exact(device, m, n, k):
    """-128 included (the reference's generators stop at -127): the int32 result is exact."""
    rng = np.random.default_rng(m * n + k)
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    b = rng.integers(-128, 128, (n, k), dtype=np.int8)
    a[0, :] = -128
    b[0, :] = -128
    c = device.empty(T.i32, m, n)
    programs.gemm_i8_i32[TILING](device.to_device(a), device.to_device(b), c)
    np.testing.assert_array_equal(c.to_host(), a.astype(np.int64) @ b.astype(np.int64).T)


# one shape per kernel family whose whole blocks take the direct store: the mid-size pipeline (512^3), the
# four-wave whole-tile loop (4096 x 4096 x 256) and the eight-wave int8 pipeline (W8A8-like dequantisation)
@pytest.mark.parametrize("m,n,k,dtype", [(512, 512, 512, BF16), (4096, 4096, 256, BF16), (4096, 4096, 256, I8)])
def test_direct_store_at_an_address_whose_low_word_has_bit_31_set(device, m, n, k, dtype):
    """Regression: the direct epilogue stores through a buffer resource built from the two 32-bit words of C's
    address; a low word with bit 31 set was once sign-extended into the high word (a memory fault). Here C lies at
    such an address, and its result must equal the same product into an ordinary allocation bit for bit."""
    rng = np.random.default_rng(m + k)
    if dtype == I8:
        a = device.to_device(rng.integers(-127, 128, (m, k), dtype=np.int8))
        b = device.to_device(rng.integers(-127, 128, (n, k), dtype=np.int8))
        sa = device.to_device(rng.uniform(0.5, 2.0, m).astype(np.float32))
        sb = device.to_device(rng.uniform(0.5, 2.0, n).astype(np.float32))
        ops = [(library.MUL_ROW, 0.0, sa.pointer), (library.MUL_COL, 0.0, sb.pointer)]
    else:
        a = device.to_device(bf16_words(rng.standard_normal((m, k)).astype(np.float32)), T.bf16)
        b = device.to_device(bf16_words(rng.standard_normal((n, k)).astype(np.float32)), T.bf16)
        ops = []
    nbytes = m * n * 2
    want = device.empty(T.bf16, m, n)
    stream = device.default_stream.handle
    library.gemm_nt(dtype, a.pointer, b.pointer, want.pointer, BF16, m, n, k, ops, stream)
    arena = device.empty(T.u8, (1 << 31) + nbytes + 256)
    low = arena.pointer & 0xFFFFFFFF
    offset = 0 if low >= 0x80000000 else (0x80000000 - low + 255) // 256 * 256
    target = arena.pointer + offset
    assert target & 0x80000000 and offset + nbytes <= (1 << 31) + nbytes + 256
    library.gemm_nt(dtype, a.pointer, b.pointer, target, BF16, m, n, k, ops, stream)
    device.default_stream.sync()
    got = np.empty((m, n), np.uint16)
    hipapi.api().hipMemcpy(got.ctypes.data, target, nbytes, hipapi.D2H)
    np.testing.assert_array_equal(got, want.to_host())


# The four-wave whole-tile loop (at least 128 tiles of 256 x 256) runs its slices two at a time; these K give the
# fewest slices it takes (2), an odd count (3, the tail slice) and 5, for bf16, f16 and fp8, with ragged M and N.
@pytest.mark.parametrize("k_slices", [2, 3, 5])
@pytest.mark.parametrize("dtype", ["bf16", "f16", "fp8"])
def test_four_wave_loop_at_its_slice_counts(device, dtype, k_slices):
    m, n = 4096 - 40, 2048 + 256 * 4 - 24  # 16 x 12 = 192 tiles, the last row and column ragged
    rng = np.random.default_rng(k_slices * 10 + len(dtype))
    rows = np.r_[0:64, m - 64:m]  # the first and the last (ragged) row tiles, all columns
    if dtype == "fp8":
        k = 128 * k_slices
        a = e4m3_encode(rng.standard_normal((m, k)).astype(np.float32))
        b = e4m3_encode(rng.standard_normal((n, k)).astype(np.float32))
        c = device.empty(T.bf16, m, n)
        sa, sb = 0.5, 0.25
        programs.gemm_fp8[programs.Tiling(bm=64, bn=64, bk=64)](
            device.to_device(a, T.f8e4m3fn), device.to_device(b, T.f8e4m3fn), c, sa, sb)
        got = bf16_values(c.to_host()[rows]).astype(np.float64)
        da, db = e4m3_decode(a[rows]).astype(np.float64), e4m3_decode(b).astype(np.float64)
        scale = np.float64(np.float32(sa * sb))
        reference = (da @ db.T) * scale
        bound = (8 * 2.0**-24 * (k + 8) * (np.abs(da) @ np.abs(db).T)) * scale + np.abs(reference) * 2.0**-8 * 1.01
        assert np.all(np.abs(got - reference) <= bound + 1e-30)
        return
    k = 64 * k_slices
    x, y = rng.standard_normal((m, k)).astype(np.float32), rng.standard_normal((n, k)).astype(np.float32)
    if dtype == "bf16":
        aw, bw, kind = bf16_words(x), bf16_words(y), T.bf16
        av, bv = bf16_values(aw), bf16_values(bw)
    else:
        aw, bw, kind = x.astype(np.float16), y.astype(np.float16), T.f16
        av, bv = aw.astype(np.float32), bw.astype(np.float32)
    c = device.empty(kind, m, n)
    if dtype == "bf16":  # krn's program
        programs.gemm_nt[TILING](device.to_device(aw, kind), device.to_device(bw, kind), c)
    else:  # the C ABI (no f16 NT program among the test programs)
        da, db = device.to_device(aw, kind), device.to_device(bw, kind)
        library.gemm_nt(F16, da.pointer, db.pointer, c.pointer, F16, m, n, k, [], device.default_stream.handle)
    out = c.to_host()[rows]
    got = bf16_values(out) if dtype == "bf16" else out.astype(np.float32)
    assert_agrees(got, av[rows], bv.T, k, dtype)


def test_w8a8_with_a_half_empty_last_wave_splits_its_columns_bit_exactly(device):
    """4096 x 4352: 272 tiles of 256 x 256, a last wave of 16 on 256 CUs. The first 4096 columns (256 tiles, one
    full wave) run as 256 x 256 tiles and the last 256 as 128 x 256 tiles in a second launch, whose per-column
    scale vector starts at column 4096. int32 accumulation is exact: bf16(f32(f32(acc) * sa[m]) * sw[n])."""
    m, n, k = 4096, 4352, 128
    rng = np.random.default_rng(61)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    sa = (rng.uniform(0.5, 1.5, (m, 1)) / 127).astype(np.float32)
    sw = (rng.uniform(0.5, 1.5, (1, n)) / 127).astype(np.float32)
    c = device.empty(T.bf16, m, n)
    programs.gemm_w8a8[programs.Tiling(bm=256, bn=256, bk=128)](device.to_device(a), device.to_device(w),
                                                               device.to_device(sa), device.to_device(sw), c)
    acc = (a.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32)
    np.testing.assert_array_equal(c.to_host(), bf16_words((acc * sa).astype(np.float32) * sw))


def test_bf16_with_a_half_empty_last_wave_and_a_column_bias(device):
    """The same column split for bf16 with a per-column f32 bias added into an f32 result: each column's bias
    lands on its own column in both launches (within the accumulation bound of float64)."""
    m, n, k = 4096, 4352, 256
    rng = np.random.default_rng(62)
    aw, bw = (bf16_words(rng.standard_normal(s).astype(np.float32)) for s in ((m, k), (n, k)))
    bias = rng.standard_normal(n).astype(np.float32)
    a, b, dbias = device.to_device(aw, T.bf16), device.to_device(bw, T.bf16), device.to_device(bias)
    c = device.empty(T.f32, m, n)
    library.gemm_nt(BF16, a.pointer, b.pointer, c.pointer, F32, m, n, k, [(library.ADD_COL, 0.0, dbias.pointer)],
                    device.default_stream.handle)
    reference, bound = agree_bound(bf16_values(aw), bf16_values(bw).T, k)
    want = reference + bias.astype(np.float64)
    assert np.all(np.abs(c.to_host().astype(np.float64) - want) <= bound + np.abs(want) * 2.0**-24)

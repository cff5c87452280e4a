"""The oracle pinned: every function of oracle/ is checked against what fixes it independently of its own formula
-- closed forms, exhaustive tables, exact rational arithmetic, brute force -- chosen so that a dropped term, a wrong
rounding direction or a transposed operand fails. Also the product's host conversions against the oracle's."""

import math
from fractions import Fraction

import numpy as np
import pytest

from krn_amd import formats
from krn_amd.compiler.capture import capture
from krn_amd.frontend import Blocks
from oracle import cbackend, emulate, numerics
from tests.conftest import KERNELS
from tests.helpers import assert_agrees


# ---- bf16 ------------------------------------------------------------------------------------------------------


def test_bf16_rounding_known_answers():
    cases = {
        0x3F800000: 0x3F80,  # 1.0 exact
        0x3F808000: 0x3F80,  # tie, even stays
        0x3F818000: 0x3F82,  # tie, odd rounds up
        0x3F808001: 0x3F81,  # just above the tie
        0x3F807FFF: 0x3F80,  # just below the tie
        0x7F7FFFFF: 0x7F80,  # largest float rounds to infinity
        0x7F800000: 0x7F80,  # infinity
        0xFF800000: 0xFF80,  # -infinity
        0x7FC00001: 0x7FC0,  # quiet NaN keeps being NaN
        0x7F800001: 0x7FC0,  # signalling NaN becomes quiet
        0x00000001: 0x0000,  # smallest subnormal rounds to zero
        0x80000000: 0x8000,  # -0.0
    }
    words = np.array(list(cases), np.uint32).view(np.float32)
    got = numerics.bf16_words(words)
    np.testing.assert_array_equal(got, np.array(list(cases.values()), np.uint16))
    np.testing.assert_array_equal(formats.bf16_words(words), got)


def test_bf16_rounding_is_the_nearest_even_of_its_two_neighbours():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(20000) * 10.0 ** rng.integers(-30, 30, 20000)).astype(np.float32)
    got = numerics.bf16_round(x).astype(np.float64)
    bits = x.view(np.uint32)
    low = (bits & np.uint32(0xFFFF0000)).view(np.float32).astype(np.float64)
    high = ((bits & np.uint32(0xFFFF0000)) + np.uint32(0x10000)).view(np.float32).astype(np.float64)
    xd = x.astype(np.float64)
    d_low, d_high = np.abs(xd - low), np.abs(high - xd)
    even_low = ((bits >> 16) & 1) == 0
    want = np.where(d_low < d_high, low, np.where(d_high < d_low, high, np.where(even_low, low, high)))
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(formats.bf16_words(x), numerics.bf16_words(x))


# ---- fp8 e4m3fn --------------------------------------------------------------------------------------------------


def test_e4m3_table_known_values():
    t = numerics.TABLE
    assert t[0x00] == 0 and t[0x01] == 2.0**-9 and t[0x07] == 7 * 2.0**-9 and t[0x08] == 2.0**-6
    assert t[0x38] == 1.0 and t[0x39] == 1.125 and t[0x7E] == 448.0 and np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    assert t[0xB8] == -1.0 and t[0x80] == 0 and np.signbit(t[0x80])
    finite = t[np.isfinite(t)]
    assert len(finite) == 254 and len(set(np.abs(finite).tolist())) == 127  # +-0 and 126 other magnitudes


def exact_code(x: float) -> int:
    """Brute force over all finite codes with exact rationals: nearest value, ties to the even code, saturating."""
    if math.isnan(x):
        return 0x7F
    sign = 0x80 if math.copysign(1.0, x) < 0 else 0
    magnitude = Fraction(min(abs(x), 448.0))
    best = min(range(0x7F), key=lambda c: (abs(Fraction(float(numerics.TABLE[c])) - magnitude), c % 2))
    return sign | best


def e4m3_inputs(seed: int) -> np.ndarray:
    table = numerics.TABLE[np.isfinite(numerics.TABLE)].astype(np.float32)
    levels = np.unique(np.abs(table.astype(np.float64)))
    mids = ((levels[:-1] + levels[1:]) / 2).astype(np.float32)
    near = np.concatenate([mids.view(np.uint32) + np.uint32(s) for s in (0, 1, 0xFFFFFFFF)]).view(np.float32)
    rng = np.random.default_rng(seed)
    random = (rng.standard_normal(2000) * 300).astype(np.float32)
    special = np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 1e30, -1e30, 2.0**-10, 3 * 2.0**-10, 449.0, 464.0, 465.0],
                       np.float32)
    return np.concatenate([table, near, -near, random, special])


def test_e4m3_encoders_match_the_exact_rational_search():
    x = e4m3_inputs(5)
    want = np.array([exact_code(float(v)) for v in x], np.uint8)
    np.testing.assert_array_equal(numerics.e4m3_encode(x), want)
    np.testing.assert_array_equal(formats.e4m3_encode(x), want)
    np.testing.assert_array_equal([numerics.e4m3_encode_one(float(v)) for v in x[:300]], want[:300])


def test_every_finite_e4m3_code_round_trips():
    codes = np.arange(256, dtype=np.uint8)
    values = numerics.e4m3_decode(codes)
    live = np.isfinite(values)
    np.testing.assert_array_equal(numerics.e4m3_encode(values[live]), codes[live])
    np.testing.assert_array_equal(formats.e4m3_decode(codes)[live], values[live])


# ---- fused multiply-add ------------------------------------------------------------------------------------------


def exact_fma(a: float, b: float, c: float) -> np.float32:
    """float32 rounding of the exact rational a*b + c (ties to even): the definition of a fused multiply-add."""
    value = Fraction(a) * Fraction(b) + Fraction(c)
    candidate = np.float32(float(value))  # float64 rounding first, then the exact decision below
    below = np.nextafter(candidate, np.float32(-np.inf))
    above = np.nextafter(candidate, np.float32(np.inf))
    best = min((candidate, below, above), key=lambda v: (abs(Fraction(float(v)) - value),
                                                       int(np.float32(v).view(np.uint32)) & 1))
    return np.float32(best)


def test_fma32_is_the_single_rounding_of_the_exact_result():
    rng = np.random.default_rng(3)
    a = rng.standard_normal(3000).astype(np.float32)
    b = rng.standard_normal(3000).astype(np.float32)
    c = rng.standard_normal(3000).astype(np.float32)
    # adversarial: c cancels most of a*b, so a two-rounding a*b + c differs
    c[:1000] = -(a[:1000].astype(np.float64) * b[:1000]).astype(np.float32)
    got = numerics.fma32(a, b, c)
    want = np.array([exact_fma(float(x), float(y), float(z)) for x, y, z in zip(a, b, c)], np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    two_roundings = (a * b + c).astype(np.float32)
    assert (two_roundings != want).any()  # the check can tell a fused result from an unfused one


# ---- emulator and C backend --------------------------------------------------------------------------------------


def test_c1_f32_gemm_is_bit_identical_between_emulator_and_c_backend_and_within_the_bound():
    """f32 256^3, A and B ~ U[-1, 1] from a seed."""
    rng = np.random.default_rng(0)
    a, b = (rng.uniform(-1, 1, (256, 256)).astype(np.float32) for _ in range(2))
    kernel = capture(KERNELS, "matmul_f32", consts={"t": {"bm": 32, "bn": 32, "bk": 16}})
    emulated, compiled = np.zeros((256, 256), np.float32), np.zeros((256, 256), np.float32)
    emulate.run(kernel, None, [a, b, emulated])
    cbackend.run(kernel, None, [a, b, compiled])
    np.testing.assert_array_equal(emulated.view(np.uint32), compiled.view(np.uint32))
    assert_agrees(compiled, a, b, 256, "f32")
    # k order matters: a reversed-k sum is a different float32 result somewhere
    reversed_sum = np.zeros_like(compiled)
    for k in reversed(range(256)):
        reversed_sum = numerics.fma32(a[:, k, None], b[None, k, :], reversed_sum)
    assert not np.array_equal(reversed_sum, compiled)


def test_c_backend_splits_the_grid_over_threads_without_changing_bits():
    rng = np.random.default_rng(1)
    a, b = (rng.uniform(-1, 1, (96, 80)).astype(np.float32), rng.uniform(-1, 1, (80, 64)).astype(np.float32))
    kernel = capture(KERNELS, "matmul_f32", consts={"t": {"bm": 32, "bn": 16, "bk": 16}})
    one, many = np.zeros((96, 64), np.float32), np.zeros((96, 64), np.float32)
    cbackend.Program(kernel)(a, b, one)
    cbackend.Program(kernel)(a, b, many, threads=4)
    np.testing.assert_array_equal(one, many)


@pytest.mark.parametrize("m,n,k,bm,bn,bk", [(50, 38, 70, 32, 32, 16), (130, 70, 100, 32, 32, 16),
                                            (16, 8, 8, 16, 8, 8), (257, 129, 33, 32, 32, 16)])
def test_oracles_agree_on_ragged_f16_products(m, n, k, bm, bn, bk):
    """krn's test_oracles (reference tests/compiler/test_tensor_cores.py:490-508): seed 1, U[-1, 1] f16."""
    rng = np.random.default_rng(1)
    a, b = (rng.uniform(-1, 1, s).astype(np.float16) for s in ((m, k), (k, n)))
    kernel = capture(KERNELS, "matmul_f16_f32", consts={"t": {"bm": bm, "bn": bn, "bk": bk}})
    emulated, compiled = np.zeros((m, n), np.float32), np.zeros((m, n), np.float32)
    emulate.run(kernel, None, [a, b, emulated])
    cbackend.run(kernel, None, [a, b, compiled])
    assert_agrees(emulated, a.astype(np.float32), b.astype(np.float32), k, "f32")
    assert_agrees(compiled, a.astype(np.float32), b.astype(np.float32), k, "f32")
    np.testing.assert_array_equal(emulated, compiled)


def numpy_attention(q, k, v, causal):
    q, k, v = (x.astype(np.float64) for x in (q, k, v))
    s = q @ k.transpose(0, 2, 1) / math.sqrt(q.shape[-1])
    if causal:
        s = np.where(np.tril(np.ones(s.shape[-2:], bool)), s, -np.inf)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    return (p / p.sum(axis=-1, keepdims=True)) @ v


@pytest.mark.parametrize("seq,heads,d,causal", [(1, 1, 8, True), (17, 2, 16, False), (40, 1, 8, True),
                                                (33, 2, 16, True)])
def test_flash_attention_on_both_oracles_matches_a_float64_softmax(seq, heads, d, causal):
    """reference tests/frontend/test_tile_ops.py:138-154: ragged sequences, atol 3e-3 against float64 numpy."""
    rng = np.random.default_rng(seq)
    q, k, v = (rng.standard_normal((heads, seq, d)).astype(np.float16) for _ in range(3))
    consts = {"bq": 8, "bk": 8, "d": d, "causal": causal}
    kernel = capture(KERNELS, "flash_attention", consts={"t": consts})
    scale = math.log2(math.e) / math.sqrt(d)
    launch = Blocks(-(-seq // 8), heads)
    want = numpy_attention(q, k, v, causal)
    for run in (emulate.run, cbackend.run):
        out = np.zeros((heads, seq, d), np.float16)
        with np.errstate(all="ignore"):
            run(kernel, launch, [q, k, v, out, scale])
        np.testing.assert_allclose(out.astype(np.float64), want, atol=3e-3)


def float64_softmax(x: np.ndarray) -> np.ndarray:
    v = x.astype(np.float64)
    e = np.exp(v - v.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


@pytest.mark.parametrize("name,rows,cols,tile_cols", [("softmax_long_rows", 6, 2500, 1024), ("softmax", 6, 512, 512),
                                                      ("softmax_steps", 5, 256, 256)])
def test_softmax_programs_on_both_oracles_match_a_float64_softmax(name, rows, cols, tile_cols):
    """krn's softmax programs (reference examples/02_tiles_and_types/01_softmax_rows.py:27-40, 44-53: 6 rows of
    2500 columns, two full chunks and a ragged one, atol 1e-3 against numpy; tests/helpers/example_softmax.py)."""
    rng = np.random.default_rng(rows + cols)
    x = (rng.standard_normal((rows, cols)) * 4).astype(np.float16)
    kernel = capture(KERNELS, name, consts={"t": {"rows": 4, "cols": tile_cols}})
    want = float64_softmax(x.astype(np.float32))
    for run in (emulate.run, cbackend.run):
        y = np.zeros((rows, cols), np.float16)
        run(kernel, Blocks(-(-rows // 4)), [x, y])
        np.testing.assert_allclose(y.astype(np.float64), want, atol=1e-3)


def test_int8_products_accumulate_exactly_in_int32_on_both_oracles():
    rng = np.random.default_rng(4)
    a = rng.integers(-127, 128, (33, 70), dtype=np.int8)
    w = rng.integers(-127, 128, (20, 70), dtype=np.int8)
    kernel = capture(KERNELS, "gemm_i8_i32", consts={"t": {"bm": 16, "bn": 16, "bk": 16}})
    want = a.astype(np.int64) @ w.astype(np.int64).T
    for run in (emulate.run, cbackend.run):
        out = np.zeros((33, 20), np.int32)
        run(kernel, None, [a, w, out])
        np.testing.assert_array_equal(out, want)


def test_fp8_products_decode_exactly_on_both_oracles():
    rng = np.random.default_rng(5)
    a = numerics.e4m3_encode(rng.standard_normal((24, 64)).astype(np.float32) * 8)
    b = numerics.e4m3_encode(rng.standard_normal((40, 64)).astype(np.float32) * 8)
    kernel = capture(KERNELS, "gemm_fp8", consts={"t": {"bm": 16, "bn": 16, "bk": 32}})
    outs = []
    for run in (emulate.run, cbackend.run):
        out = np.zeros((24, 40), np.uint16)
        run(kernel, None, [a, b, out, np.float32(0.5), np.float32(0.25)])
        outs.append(out)
    np.testing.assert_array_equal(outs[0], outs[1])
    da, db = numerics.e4m3_decode(a).astype(np.float64), numerics.e4m3_decode(b).astype(np.float64)
    reference = (da @ db.T) * 0.125
    got = numerics.bf16_values(outs[0]).astype(np.float64)
    assert np.all(np.abs(got - reference) <= np.abs(reference) * 2.0**-8 + 1e-12 + 8 * 2.0**-24 * 72 * 0.125 *
                  (np.abs(da) @ np.abs(db).T))

"""Number formats of the oracle: bfloat16 rounding, the e4m3fn fp8 codec and the single-rounding float32 FMA.

TEST INFRASTRUCTURE ONLY. Nothing under `oracle/` is part of the product: only `tests/`, `__graft_entry__.smoke()` and
`bench.py`'s CPU-baseline leg may import it, and only as the checker.

Each function restates krn's definition and is pinned by a check in tests/test_oracle.py that a plausible mistake
would fail (closed forms, exhaustive code tables, exact rational search, brute force).
"""

from fractions import Fraction

import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), kept in float32 storage; a NaN stays NaN and becomes quiet.
    Follows reference src/krn/emulator/emulate.py:144-150 (and the HIP text compiler/hip.py:123-130)."""
    bits = np.asarray(x, np.float32).view(np.uint32)
    lsb = (bits >> np.uint32(16)) & np.uint32(1)
    rounded = (bits + np.uint32(0x7FFF) + lsb) & np.uint32(0xFFFF0000)
    quiet = (bits | np.uint32(0x00400000)) & np.uint32(0xFFFF0000)
    nan = (bits & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    return np.where(nan, quiet, rounded).view(np.float32)


def bf16_words(x: np.ndarray) -> np.ndarray:
    """The uint16 storage words of bf16_round(x)."""
    return (bf16_round(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def bf16_values(words: np.ndarray) -> np.ndarray:
    return (np.asarray(words, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def e4m3_table() -> np.ndarray:
    """The float64 value of each of the 256 e4m3fn codes: bias 7, subnormals at exponent field 0, S.1111.111 is NaN
    and there are no infinities (OCP fp8; the same formula as reference tests/compiler/test_tensor_cores.py:200-216)."""
    values = np.zeros(256, np.float64)
    for code in range(256):
        mantissa, exponent = code & 7, (code >> 3) & 15
        if exponent == 0:
            value = mantissa / 8 * 2.0 ** (1 - 7)
        else:
            value = (1 + mantissa / 8) * 2.0 ** (exponent - 7)
        if code & 0x7F == 0x7F:
            value = np.nan
        values[code] = -value if code & 0x80 else value
    return values


TABLE = e4m3_table()
_POSITIVE = [(Fraction(float(TABLE[c])), c) for c in range(0x7F)]  # every finite non-negative code 0..0x7E
E4M3_MAX = 448.0


def e4m3_encode_one(x: float) -> int:
    """The code of one float32 value: nearest finite value, ties to the even code, saturating at +-448, NaN to
    0x7F, the sign kept for zero (reference compiler/narrow.py:94-105, pinned there by tests/compiler/
    test_narrow.py:74-112's exact rational search, which this is)."""
    x = float(np.float32(x))
    if np.isnan(x):
        return 0x7F
    sign = 0x80 if np.signbit(x) else 0
    magnitude = Fraction(min(abs(x), E4M3_MAX))
    _, code = min(((abs(v - magnitude), c % 2), c) for v, c in _POSITIVE)
    return sign | code


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """Vectorized e4m3_encode_one: midpoints between neighbouring codes decide, ties go to the even code."""
    x = np.asarray(x, np.float32)
    flat = x.reshape(-1).astype(np.float64)
    levels = TABLE[:0x7F]  # increasing non-negative finite values
    magnitude = np.minimum(np.abs(flat), E4M3_MAX)
    above = np.searchsorted(levels, magnitude, side="left").clip(0, 0x7E)  # first level >= magnitude
    below = np.maximum(above - 1, 0)
    d_above, d_below = levels[above] - magnitude, magnitude - levels[below]
    code = np.where(d_below < d_above, below, above)
    tie = (d_below == d_above) & (above != below)
    code = np.where(tie, np.where(below % 2 == 0, below, above), code)
    sign = np.where(np.signbit(flat), 0x80, 0)
    out = (sign | code).astype(np.uint8)
    out[np.isnan(flat)] = 0x7F
    return out.reshape(x.shape)


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    return TABLE[np.asarray(codes, np.uint8)].astype(np.float32)


def fma32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """a * b + c in float32 with one rounding, elementwise, for finite inputs.

    The product of two float32 values is exact in float64. The float64 sum is then rounded to odd: if the TwoSum
    error is nonzero and the sum's last bit is even, step one ulp towards the error. Rounding that to float32 is the
    correctly rounded fused result, because float64 carries more than 24 + 2 bits (Boldo & Melquiond, "Emulation of
    FMA and correctly rounded sums: proved algorithms using rounding to odd", IEEE TC 2008). The reference emulator
    uses the same construction (src/krn/emulator/emulate.py:347-385)."""
    a, b, c = (np.asarray(v, np.float64) for v in (a, b, c))
    p = a * b
    s = p + c
    bp = s - p
    err = (p - (s - bp)) + (c - bp)
    odd = (s.view(np.int64) & 1).astype(bool)
    s = np.where((err != 0) & ~odd, np.nextafter(s, np.where(err > 0, np.inf, -np.inf)), s)
    with np.errstate(over="ignore"):
        return s.astype(np.float32)

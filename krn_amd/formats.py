"""Host-side storage conversions of the tile path: float32 -> bf16 words and float32 -> fp8 e4m3fn codes.

krn stores bf16 tensors as raw uint16 words and fp8 tensors as uint8 codes (reference README;
src/krn/data/formats.py:95 E4M3FN; src/krn/compiler/narrow.py:94-105 reference_encode). These are what a caller uses
to prepare device tensors, for example the per-tensor quantization `codes = e4m3(x / (amax / 448))`.
"""

import numpy as np

E4M3_MAX = 448.0


def bf16_words(x: np.ndarray) -> np.ndarray:
    """Nearest bfloat16 (ties to even) as uint16 words; a NaN keeps its sign and becomes quiet."""
    bits = np.asarray(x, np.float32).view(np.uint32)
    nan = (bits & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    rounded = (bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    quiet = (bits | np.uint32(0x00400000)) >> np.uint32(16)
    return np.where(nan, quiet, rounded).astype(np.uint16)


def bf16_values(words: np.ndarray) -> np.ndarray:
    return (np.asarray(words, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn code: nearest representable value with ties to the even code, magnitudes above 448
    (infinities included) saturate to +-448, NaN becomes 0x7F, and the sign of zero is kept."""
    x = np.asarray(x, np.float32)
    a = np.abs(x).astype(np.float64)
    nan = np.isnan(a)
    a = np.minimum(np.where(nan, 0.0, a), E4M3_MAX)
    # subnormals: multiples of 2^-9 below 2^-6
    sub = np.rint(a * 512.0)  # ties to even
    mantissa, exponent = np.frexp(a)  # a = mantissa * 2^exponent, mantissa in [0.5, 1)
    e = exponent - 1  # a = (2 * mantissa) * 2^e with 2 * mantissa in [1, 2)
    m3 = np.rint((2.0 * mantissa - 1.0) * 8.0)
    carry = m3 == 8
    e, m3 = np.where(carry, e + 1, e), np.where(carry, 0, m3)
    normal = ((e + 7).astype(np.int64) << 3) | m3.astype(np.int64)
    code = np.where(a < 2.0**-6, sub.astype(np.int64), normal)  # sub == 8 is the smallest normal, code 0x08
    code = np.minimum(code, 0x7E)
    code = code | np.where(np.signbit(x), 0x80, 0)
    code = np.where(nan, 0x7F, code)
    return code.astype(np.uint8)


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """e4m3fn code -> float32 value (S.1111.111 is NaN; there are no infinities)."""
    c = np.asarray(codes, np.uint8).astype(np.int64)
    m, e = c & 7, (c >> 3) & 15
    value = np.where(e == 0, m / 8.0 * 2.0**-6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    value = np.where((c & 0x7F) == 0x7F, np.nan, value)
    return np.where(c & 0x80, -value, value).astype(np.float32)

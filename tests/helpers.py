"""Shared test helpers: seeded inputs in krn's storage forms and the accumulation-order-free error bound."""

import numpy as np

from oracle.numerics import bf16_values, bf16_words


def agree_bound(a: np.ndarray, b: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """The float64 product and krn's forward-error bound for a float32-accumulated product of k terms in any order
    (reference tests/compiler/test_tensor_cores.py:395-401): |C - A.B| <= 8 * 2^-24 * (k + 8) * (|A|.|B|)."""
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    return a64 @ b64, 8 * 2.0**-24 * (k + 8) * (np.abs(a64) @ np.abs(b64))


def assert_agrees(actual: np.ndarray, a: np.ndarray, b: np.ndarray, k: int, output: str) -> None:
    """`actual` (f32 values, or bf16/f16 results widened) within the bound, plus one output rounding for 16-bit
    outputs: 2^-8 relative for bf16, f16's own spacing for f16."""
    reference, bound = agree_bound(a, b, k)
    if output == "bf16":
        bound = bound + np.abs(reference) * 2.0**-8 + 2.0**-133
    elif output == "f16":
        bound = bound + np.abs(reference.astype(np.float16).astype(np.float64) - reference)
        bound = bound + np.spacing(np.abs(reference).astype(np.float16)).astype(np.float64)
    error = np.abs(actual.astype(np.float64) - reference)
    worst = np.unravel_index(np.argmax(error - bound), error.shape)
    assert np.all(error <= bound), f"error {error[worst]} > bound {bound[worst]} at {worst}"


def bf16_normal(rng: np.random.Generator, shape: tuple[int, ...]) -> tuple[np.ndarray, np.ndarray]:
    """N(0, 1) values rounded to bf16: (uint16 words, their float32 values)."""
    words = bf16_words(rng.standard_normal(shape).astype(np.float32))
    return words, bf16_values(words)

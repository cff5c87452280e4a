"""The four-wave whole-tile loop's direct stores (16-bit and float32 outputs) with epilogue chains, bit for bit.

gemm_quad16 computes its blocks transposed and stores them straight from the accumulators, applying each operation
of the chain as fused multiply-adds (x * s + (-0) for a multiply, x * 1 + s for an add, and the identity
x * 1 + (-0) for the other of the pair). That must equal the patch path's arithmetic exactly: every operation
rounded once to float32, in order, then one rounding to the 16-bit output. int8 operands make the accumulators
exact (int32), so the expected output is computed here in numpy float32, which rounds each multiply and add
correctly. The products have 128 tiles of 256 x 256 (the dispatch's whole-tile loop) with whole tiles, so every
wave takes the direct store; rows of zeros in A give zero accumulators, which check the signed zeros (x * -1 = -0,
0 + (-0) = +0)."""

import numpy as np
import pytest

from krn_amd import T
from krn_amd.dtypes import BF16, F16, F32, I8
from krn_amd.runtime import library
from oracle.numerics import bf16_words

pytestmark = pytest.mark.gpu

M, N, K = 2048, 4096, 512
F32_KIND, F16_KIND, BF16_KIND = 0, 1, 2


def _vector_bits(values: np.ndarray, kind: int) -> np.ndarray:
    if kind == F32_KIND:
        return values.astype(np.float32)
    if kind == F16_KIND:
        return values.astype(np.float16)
    return bf16_words(values.astype(np.float32))


def _vector_values(values: np.ndarray, kind: int) -> np.ndarray:
    """What the kernel reads back from a vector of this kind, as float32."""
    if kind == F32_KIND:
        return values.astype(np.float32)
    if kind == F16_KIND:
        return values.astype(np.float16).astype(np.float32)
    return (bf16_words(values.astype(np.float32)).astype(np.uint32) << 16).view(np.float32)


# (operation, vector kind, scalar) chains; the vectors are drawn per test
CHAINS = [
    [(library.ADD_ROW, F32_KIND, 0.0), (library.MUL_SCALAR, 0, -0.75)],
    [(library.MUL_COL, BF16_KIND, 0.0), (library.ADD_SCALAR, 0, -0.0)],
    [(library.ADD_COL, F16_KIND, 0.0), (library.ADD_ROW, F32_KIND, 0.0)],
    [(library.MUL_ROW, F32_KIND, 0.0), (library.MUL_COL, F32_KIND, 0.0)],
    [(library.MUL_SCALAR, 0, -1.0)],
    [],
]


@pytest.mark.parametrize("out", [BF16, F16, F32])
@pytest.mark.parametrize("chain", range(len(CHAINS)))
def test_direct_store_chain_is_bit_exact(device, chain, out):
    rng = np.random.default_rng(500 + chain)
    # small integers keep every result finite in f16 (|acc| <= 64 K = 32768, plus at most 8192 from an add)
    a = rng.integers(-8, 9, (M, K), dtype=np.int8)
    a[::97] = 0  # zero accumulators in these rows
    b = rng.integers(-8, 9, (N, K), dtype=np.int8)
    want = (a.astype(np.int64) @ b.astype(np.int64).T).astype(np.float32)
    ops, keep = [], []
    for op, kind, scalar in CHAINS[chain]:
        code = op | (kind << 4)
        if op in (library.MUL_SCALAR, library.ADD_SCALAR):
            s = np.float32(scalar)
            want = want * s if op == library.MUL_SCALAR else want + s
            ops.append((code, float(scalar), None))
            continue
        per_row = op in (library.MUL_ROW, library.ADD_ROW)
        length = M if per_row else N
        raw = rng.uniform(-2.0, 2.0, length) * (2.0**-12 if op in (library.MUL_ROW, library.MUL_COL) else 4096.0)
        vec = device.to_device(_vector_bits(raw, kind))
        keep.append(vec)
        vals = _vector_values(raw, kind)
        vals = vals[:, None] if per_row else vals[None, :]
        want = want * vals if op in (library.MUL_ROW, library.MUL_COL) else want + vals
        want = want.astype(np.float32)
        ops.append((code, 0.0, vec.pointer))
    c = device.empty({BF16: T.bf16, F16: T.f16, F32: T.f32}[out], M, N)
    library.gemm_nt(I8, device.to_device(a).pointer, device.to_device(b).pointer, c.pointer, out, M, N, K, ops,
                    device.default_stream.handle)
    got = c.to_host()
    if out == F32:
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        return
    expect = bf16_words(want) if out == BF16 else want.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got.view(np.uint16), expect)

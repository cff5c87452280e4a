"""krn_gemm_nn_noalloc, the NN product for callers that cannot allocate (code under graph capture, serving loops,
harnesses that forbid hipMalloc): the transposed operand lives in the library's own device array instead of a
workspace. Called through the C ABI and checked bit for bit against krn_gemm_nn with a workspace, on two calls in a
row, the second smaller, and refused beyond its limit."""

import numpy as np
import pytest

from krn_amd import T
from krn_amd.dtypes import BF16, F16
from krn_amd.runtime import library
from oracle.numerics import bf16_words

pytestmark = pytest.mark.gpu


def operands(device, rng, dtype, m, n, k):
    x, y = rng.standard_normal((m, k)).astype(np.float32), rng.standard_normal((k, n)).astype(np.float32)
    if dtype == BF16:
        return device.to_device(bf16_words(x), T.bf16), device.to_device(bf16_words(y), T.bf16), T.bf16
    return device.to_device(x.astype(np.float16)), device.to_device(y.astype(np.float16)), T.f16


def with_workspace(device, dtype, a, b, c, m, n, k, ops=(), vectors=()):
    need = library.gemm_nn_workspace(n, k)
    workspace = device.empty(T.u8, max(need, 1))
    codes, scalars, vecs = library.marshal_ops([(op, 0.0, v) for op, v in zip(ops, vectors)])
    library.check(library.lib().krn_gemm_nn(library.kind(dtype), a.pointer, b.pointer, c.pointer, library.kind(dtype),
                                            m, n, k, len(ops), codes, scalars, vecs, workspace.pointer, max(need, 1),
                                            device.default_stream.handle), "krn_gemm_nn")
    device.default_stream.sync()


def no_alloc(device, dtype, a, b, c, m, n, k, ops=(), vectors=()):
    codes, scalars, vecs = library.marshal_ops([(op, 0.0, v) for op, v in zip(ops, vectors)])
    library.check(library.lib().krn_gemm_nn_noalloc(library.kind(dtype), a.pointer, b.pointer, c.pointer,
                                                    library.kind(dtype), m, n, k, len(ops), codes, scalars, vecs,
                                                    device.default_stream.handle), "krn_gemm_nn_noalloc")
    device.default_stream.sync()


@pytest.mark.parametrize("dtype", [BF16, F16])
def test_no_alloc_nn_product_matches_the_workspace_entry_point_twice(device, dtype):
    rng = np.random.default_rng(77)
    # the second call is smaller: the array keeps the first call's transposed operand, which must not leak into it
    for m, n, k in [(512, 1536, 1024), (130, 200, 96)]:
        a, b, kind = operands(device, rng, dtype, m, n, k)
        want, got = device.empty(kind, m, n), device.empty(kind, m, n)
        with_workspace(device, dtype, a, b, want, m, n, k)
        no_alloc(device, dtype, a, b, got, m, n, k)
        np.testing.assert_array_equal(got.to_host(), want.to_host(), err_msg=f"{m}x{n}x{k}")


def test_no_alloc_nn_product_with_an_epilogue(device):
    rng = np.random.default_rng(78)
    m, n, k = 256, 384, 512
    a, b, kind = operands(device, rng, F16, m, n, k)
    bias = device.to_device(rng.standard_normal(n).astype(np.float16))
    ops = (library.ADD_COL + library.VECTOR_KINDS[F16], library.GELU)
    want, got = device.empty(kind, m, n), device.empty(kind, m, n)
    with_workspace(device, F16, a, b, want, m, n, k, ops, (bias.pointer, 0))
    no_alloc(device, F16, a, b, got, m, n, k, ops, (bias.pointer, 0))
    np.testing.assert_array_equal(got.to_host(), want.to_host())


def test_no_alloc_nn_product_refuses_operands_beyond_its_scratch(device):
    limit = library.lib().krn_gemm_nn_noalloc_limit()
    assert limit == 64 << 20
    n = 8192
    k = limit // (2 * n) + 1  # one row of B too many
    a, b = device.empty(T.bf16, 16, k), device.empty(T.bf16, k, n)
    c = device.empty(T.bf16, 16, n)
    code = library.lib().krn_gemm_nn_noalloc(library.kind(BF16), a.pointer, b.pointer, c.pointer, library.kind(BF16),
                                             16, n, k, 0, None, None, None, device.default_stream.handle)
    assert code != 0 and b"scratch" in library.lib().krn_amd_last_error()


def test_no_alloc_nn_product_of_a_large_b_read_as_it_lies(device):
    """A B of 69 MB, beyond the 64 MiB array: the kernel reads it K x N as it lies, so the no-alloc entry point takes
    it (no scratch is used) and equals the NT product on B transposed on the host bit for bit; then a smaller call
    through the array (the transposed path) right after it."""
    rng = np.random.default_rng(79)
    m, n, k = 2048, 8192, 4224
    assert n * k * 2 > library.lib().krn_gemm_nn_noalloc_limit()
    assert library.gemm_nn_workspace_for(1 << 20, 1 << 20, m, n, k) == 0
    x, y = rng.standard_normal((m, k)).astype(np.float32), rng.standard_normal((k, n)).astype(np.float32)
    aw, bw = bf16_words(x), bf16_words(y)
    a, b = device.to_device(aw, T.bf16), device.to_device(bw, T.bf16)
    bt = device.to_device(np.ascontiguousarray(bw.T), T.bf16)
    want, got = device.empty(T.bf16, m, n), device.empty(T.bf16, m, n)
    library.gemm_nt(BF16, a.pointer, bt.pointer, want.pointer, BF16, m, n, k, [], device.default_stream.handle)
    no_alloc(device, BF16, a, b, got, m, n, k)
    np.testing.assert_array_equal(got.to_host(), want.to_host())
    m, n, k = 130, 200, 96
    a, b, kind = operands(device, rng, BF16, m, n, k)
    want, got = device.empty(kind, m, n), device.empty(kind, m, n)
    with_workspace(device, BF16, a, b, want, m, n, k)
    no_alloc(device, BF16, a, b, got, m, n, k)
    np.testing.assert_array_equal(got.to_host(), want.to_host())

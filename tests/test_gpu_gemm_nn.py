"""krn_gemm_nn, the NN product of krn's own GEMM example (reference examples/04_libraries/01_gemm_tiles.py:34-40,
B stored K x N), through the C ABI. Large products with N % 256 == 0 and K % 64 == 0 read B K-major as it lies
(transposed LDS reads), the others transpose B into the caller's workspace and run the NT kernels; either way the
result is bit-identical to krn_gemm_nt on B transposed on the host, because every lane pairs the same k in the same
order. A workspace that is too small is refused before anything is enqueued when the product needs one."""


import ctypes

import numpy as np
import pytest

from krn_amd import T
from krn_amd.dtypes import BF16, F16, F32
from krn_amd.runtime import library
from oracle.numerics import bf16_words

pytestmark = pytest.mark.gpu


def nt(device, dtype, a, bt, m, n, k, out):
    library.gemm_nt(dtype, a.pointer, bt.pointer, out.pointer, dtype, m, n, k, [], device.default_stream.handle)


@pytest.mark.parametrize("dtype", [BF16, F16])
@pytest.mark.parametrize("m,n,k", [(256, 512, 384), (100, 130, 72), (8, 1000, 256), (1024, 1024, 1024)])
def test_gemm_nn_equals_gemm_nt_on_the_transposed_operand(device, dtype, m, n, k):
    rng = np.random.default_rng(m + n + k)
    x, y = rng.standard_normal((m, k)).astype(np.float32), rng.standard_normal((k, n)).astype(np.float32)
    if dtype == BF16:
        ah, bh, kind = bf16_words(x), bf16_words(y), T.bf16
    else:
        ah, bh, kind = x.astype(np.float16), y.astype(np.float16), T.f16
    a, b = device.to_device(ah, kind), device.to_device(bh, kind)
    bt = device.to_device(np.ascontiguousarray(bh.T), kind)
    c_nn, c_nt = device.empty(kind, m, n), device.empty(kind, m, n)
    need = library.gemm_nn_workspace(n, k)
    assert need == n * k * 2
    workspace = device.empty(T.u8, need)
    stream = device.default_stream.handle
    library.check(library.lib().krn_gemm_nn(library.kind(dtype), a.pointer, b.pointer, c_nn.pointer,
                                            library.kind(dtype), m, n, k, 0, None, None, None, workspace.pointer,
                                            need, stream), "krn_gemm_nn")
    nt(device, dtype, a, bt, m, n, k, c_nt)
    np.testing.assert_array_equal(c_nn.to_host(), c_nt.to_host())


def operands(device, dtype, m, n, k, seed):
    rng = np.random.default_rng(seed)
    x, y = rng.standard_normal((m, k)).astype(np.float32), rng.standard_normal((k, n)).astype(np.float32)
    if dtype == BF16:
        ah, bh, kind = bf16_words(x), bf16_words(y), T.bf16
    else:
        ah, bh, kind = x.astype(np.float16), y.astype(np.float16), T.f16
    return device.to_device(ah, kind), device.to_device(bh, kind), device.to_device(np.ascontiguousarray(bh.T), kind), kind


# the direct shapes: at least 128 tiles of 256 x 256; whole and ragged M, an odd number of 128-byte K slices
@pytest.mark.parametrize("dtype", [BF16, F16])
@pytest.mark.parametrize("m,n,k", [(2048, 4096, 512), (2000, 4096, 384), (4096, 2048, 192)])
def test_gemm_nn_reading_b_as_it_lies_needs_no_workspace(device, dtype, m, n, k):
    a, b, bt, kind = operands(device, dtype, m, n, k, m + n + k)
    c_nn, c_nt = device.empty(kind, m, n), device.empty(kind, m, n)
    library.check(library.lib().krn_gemm_nn(library.kind(dtype), a.pointer, b.pointer, c_nn.pointer,
                                            library.kind(dtype), m, n, k, 0, None, None, None, None, 0,
                                            device.default_stream.handle), "krn_gemm_nn")
    nt(device, dtype, a, bt, m, n, k, c_nt)
    np.testing.assert_array_equal(c_nn.to_host(), c_nt.to_host())


def test_gemm_nn_direct_with_bias_and_activation(device):
    m, n, k = 2048, 4096, 256
    a, b, bt, kind = operands(device, BF16, m, n, k, 7)
    bias = device.to_device(np.random.default_rng(8).standard_normal(n).astype(np.float32), T.f32)
    ops = [library.ADD_COL, library.GELU]
    c_nn, c_nt = device.empty(T.f32, m, n), device.empty(T.f32, m, n)
    n_ops = len(ops)
    codes = (ctypes.c_int * n_ops)(*ops)
    scalars = (ctypes.c_float * n_ops)(0.0, 0.0)
    vectors = (ctypes.c_void_p * n_ops)(bias.pointer, None)
    stream = device.default_stream.handle
    library.check(library.lib().krn_gemm_nn(library.kind(BF16), a.pointer, b.pointer, c_nn.pointer,
                                            library.kind(F32), m, n, k, n_ops, codes, scalars, vectors, None, 0,
                                            stream), "krn_gemm_nn")
    library.check(library.lib().krn_gemm_nt(library.kind(BF16), a.pointer, bt.pointer, c_nt.pointer,
                                            library.kind(F32), m, n, k, n_ops, codes, scalars, vectors, stream),
                  "krn_gemm_nt")
    np.testing.assert_array_equal(c_nn.to_host(), c_nt.to_host())


def test_gemm_nn_refuses_a_small_workspace_and_other_kinds(device):
    m = n = k = 64
    a, b = device.empty(T.bf16, m, k), device.empty(T.bf16, k, n)
    c, workspace = device.empty(T.bf16, m, n), device.empty(T.u8, n * k * 2)
    call = library.lib().krn_gemm_nn
    assert call(library.kind(BF16), a.pointer, b.pointer, c.pointer, library.kind(BF16), m, n, k, 0, None, None, None,
                workspace.pointer, n * k * 2 - 1, None) != 0
    assert b"workspace" in library.lib().krn_amd_last_error()
    assert call(library.kind(BF16), a.pointer, b.pointer, c.pointer, library.kind(BF16), m, n, k, 0, None, None, None,
                None, 0, None) != 0
    assert call(3, a.pointer, b.pointer, c.pointer, library.kind(BF16), m, n, k, 0, None, None, None,
                workspace.pointer, n * k * 2, None) != 0  # fp8 operands: not an NN product
    assert b"bf16 or f16" in library.lib().krn_amd_last_error()


@pytest.mark.parametrize("rows,cols", [(8192, 1024), (256, 384), (128, 128), (100, 130), (129, 256), (1, 7), (300, 1)])
def test_transpose16_is_exact_on_whole_tiles_and_ragged_edges(device, rows, cols):
    """krn_transpose16 (the NN operand's transpose): whole 128 x 128 tiles take the register-transposing kernel, other
    extents the LDS-tile one; both bit-exact."""
    rng = np.random.default_rng(rows * 7 + cols)
    x = rng.integers(0, 1 << 16, (rows, cols), dtype=np.uint16)
    src, dst = device.to_device(x, T.bf16), device.empty(T.bf16, cols, rows)
    library.transpose16(src.pointer, dst.pointer, rows, cols, device.default_stream.handle)
    np.testing.assert_array_equal(dst.to_host(), x.T)

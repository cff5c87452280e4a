"""krn_gemm_nn_noalloc, the NN product for callers that cannot allocate (code under graph capture, serving loops,
harnesses that forbid hipMalloc): the transposed operand lives in the library's own device array instead of a
workspace. Called through the C ABI and checked bit for bit against krn_gemm_nn with a workspace, on two calls in a
row, the second smaller, and refused beyond its limit; it allocates nothing across calls, is ordered between two
streams that share the array, and replays correctly from a captured graph."""

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


def enqueue_no_alloc(dtype, a, b, c, m, n, k, stream_handle, ops=(), vectors=()):
    codes, scalars, vecs = library.marshal_ops([(op, 0.0, v) for op, v in zip(ops, vectors)])
    library.check(library.lib().krn_gemm_nn_noalloc(library.kind(dtype), a.pointer, b.pointer, c.pointer,
                                                    library.kind(dtype), m, n, k, len(ops), codes, scalars, vecs,
                                                    stream_handle), "krn_gemm_nn_noalloc")


def no_alloc(device, dtype, a, b, c, m, n, k, ops=(), vectors=()):
    enqueue_no_alloc(dtype, a, b, c, m, n, k, device.default_stream.handle, ops, vectors)
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


def test_no_alloc_calls_allocate_no_device_memory(device):
    """After a first call (the per-device set-up), further transposing calls leave the free device memory as it was."""
    from krn_amd.runtime import hipapi

    rng = np.random.default_rng(80)
    m, n, k = 384, 640, 768
    a, b, kind = operands(device, rng, BF16, m, n, k)
    want, got = device.empty(kind, m, n), device.empty(kind, m, n)
    with_workspace(device, BF16, a, b, want, m, n, k)
    no_alloc(device, BF16, a, b, got, m, n, k)
    device.sync()
    before = hipapi.memory_free()
    for _ in range(5):
        no_alloc(device, BF16, a, b, got, m, n, k)
    device.sync()
    assert hipapi.memory_free() == before
    np.testing.assert_array_equal(got.to_host(), want.to_host())


def test_no_alloc_calls_on_two_streams_are_ordered(device):
    """Two streams alternate transposing calls with different B operands, enqueued back to back with no host wait:
    the library makes each call wait for the previous user of the shared array, so every result is right."""
    rng = np.random.default_rng(81)
    first, second = device.stream(), device.stream()
    cases = []
    for m, n, k in [(4096, 2048, 4096), (256, 1920, 4096), (2048, 2048, 2048), (128, 384, 256)]:
        a, b, kind = operands(device, rng, F16, m, n, k)
        want, got = device.empty(kind, m, n), device.empty(kind, m, n)
        with_workspace(device, F16, a, b, want, m, n, k)
        cases.append((a, b, want, got, m, n, k))
    device.sync()
    for repeat in range(2):
        for i, (a, b, _, got, m, n, k) in enumerate(cases):
            enqueue_no_alloc(F16, a, b, got, m, n, k, (first if i % 2 == 0 else second).handle)
        first.sync()
        second.sync()
        for a, b, want, got, m, n, k in cases:
            np.testing.assert_array_equal(got.to_host(), want.to_host(), err_msg=f"{m}x{n}x{k} pass {repeat}")


def test_no_alloc_call_takes_a_stream_of_the_current_device(device):
    """The array's address is the current device's: a stream's own device must be the current one. With one GPU
    every stream matches: a created stream (not the default one) is accepted and its call is right."""
    rng = np.random.default_rng(82)
    m, n, k = 64, 128, 64
    a, b, kind = operands(device, rng, BF16, m, n, k)
    want, got = device.empty(kind, m, n), device.empty(kind, m, n)
    with_workspace(device, BF16, a, b, want, m, n, k)
    other = device.stream()
    enqueue_no_alloc(BF16, a, b, got, m, n, k, other.handle)
    other.sync()
    np.testing.assert_array_equal(got.to_host(), want.to_host())


def test_no_alloc_call_replays_from_a_captured_graph(device):
    """One transposing call recorded into a hipGraph (the caller the entry point is for) and replayed three times,
    with eager no-alloc calls on other operands and a synchronization between replays: every replay equals the
    workspace entry point."""
    rng = np.random.default_rng(83)
    m, n, k = 320, 768, 512
    a, b, kind = operands(device, rng, BF16, m, n, k)
    want, got = device.empty(kind, m, n), device.empty(kind, m, n)
    with_workspace(device, BF16, a, b, want, m, n, k)
    x, y, _ = operands(device, rng, BF16, 192, 640, 256)
    other_want, other_got = device.empty(kind, 192, 640), device.empty(kind, 192, 640)
    with_workspace(device, BF16, x, y, other_want, 192, 640, 256)
    device.sync()
    graph = device.graph(lambda: enqueue_no_alloc(BF16, a, b, got, m, n, k, device.launch_stream().handle))
    zero = np.zeros((m, n), np.uint16)
    for replay in range(3):
        got.copy_from(zero)
        device.sync()
        graph()
        device.sync()
        np.testing.assert_array_equal(got.to_host(), want.to_host(), err_msg=f"replay {replay}")
        no_alloc(device, BF16, x, y, other_got, 192, 640, 256)
        np.testing.assert_array_equal(other_got.to_host(), other_want.to_host(), err_msg=f"eager after {replay}")

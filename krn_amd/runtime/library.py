"""ctypes bindings of the C ABI of `libkrn_amd.so` (include/krn_amd.h).

Loading fails loudly: a missing library raises `LibraryNotFound`, and every nonzero return raises `KernelError`
with the library's own message. There is no fallback path.
"""

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_void_p
from functools import cache

from krn_amd.dtypes import BF16, F8E4M3, F16, F32, I8, I32, Dtype
from krn_amd.hw import Libraries

# element kinds of the C ABI (enum Kind in krn_amd/csrc/common.h)
KINDS = {F32: 0, F16: 1, BF16: 2, F8E4M3: 3, I8: 4, I32: 5}

# epilogue operations of krn_gemm_nt, applied in order with one float32 rounding each
MUL_SCALAR, MUL_ROW, MUL_COL, ADD_SCALAR, ADD_ROW, ADD_COL, RELU, GELU, SILU = range(9)
ACTIVATIONS = {"relu": RELU, "gelu": GELU, "silu": SILU}
MAX_OPS = 4  # the longest epilogue chain krn_gemm_nt takes (struct Epilogue in krn_amd/csrc/gemm.hip)
# element kind of a row/column vector, added to the operation code (float32 is 0)
VECTOR_KINDS = {F32: 0, F16: 16, BF16: 32}


class KernelError(RuntimeError):
    """A launch the gfx950 kernel library refused or failed, with its message."""


@cache
def lib() -> ctypes.CDLL:
    handle = Libraries.load("krn_amd").handle
    handle.krn_amd_last_error.restype = c_char_p
    handle.krn_amd_last_error.argtypes = []
    handle.krn_gemm_nt.restype = c_int
    handle.krn_gemm_nt.argtypes = [
        c_int, c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_int64, c_int, POINTER(c_int),
        POINTER(c_float), POINTER(c_void_p), c_void_p,
    ]  # fmt: skip
    handle.krn_attention_fwd.restype = c_int
    handle.krn_attention_fwd.argtypes = [
        c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_float, c_int, c_void_p,
    ]  # fmt: skip
    handle.krn_gemm_nn.restype = c_int
    handle.krn_gemm_nn.argtypes = [
        c_int, c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_int64, c_int, POINTER(c_int),
        POINTER(c_float), POINTER(c_void_p), c_void_p, c_int64, c_void_p,
    ]  # fmt: skip
    handle.krn_gemm_nn_workspace.restype = c_int64
    handle.krn_gemm_nn_workspace.argtypes = [c_int64, c_int64]
    handle.krn_gemm_nn_workspace_for.restype = c_int64
    handle.krn_gemm_nn_workspace_for.argtypes = [c_void_p, c_void_p, c_int64, c_int64, c_int64]
    handle.krn_gemm_nn_noalloc.restype = c_int
    handle.krn_gemm_nn_noalloc.argtypes = [
        c_int, c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int64, c_int64, c_int, POINTER(c_int),
        POINTER(c_float), POINTER(c_void_p), c_void_p,
    ]  # fmt: skip
    handle.krn_gemm_nn_noalloc_limit.restype = c_int64
    handle.krn_gemm_nn_noalloc_limit.argtypes = []
    handle.krn_transpose16.restype = c_int
    handle.krn_transpose16.argtypes = [c_void_p, c_void_p, c_int64, c_int64, c_void_p]
    handle.krn_softmax_rows.restype = c_int
    handle.krn_softmax_rows.argtypes = [c_int, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p]
    return handle


def check(code: int, what: str) -> None:
    if code != 0:
        raise KernelError(f"{what}: {lib().krn_amd_last_error().decode()} (code {code})")


def kind(dtype: Dtype) -> int:
    try:
        return KINDS[dtype]
    except KeyError:
        raise KernelError(f"{dtype} has no kind in the kernel library's C ABI") from None


def gemm_nt_call(in_dtype: Dtype, a: int, b: int, c: int, out_dtype: Dtype, m: int, n: int, k: int,
                 ops: list[tuple[int, float, int]]):
    """`gemm_nt` of these arguments as a function of the stream, with the arguments marshalled once."""
    count = len(ops)
    codes = (c_int * max(count, 1))(*(op for op, _, _ in ops))
    scalars = (c_float * max(count, 1))(*(s for _, s, _ in ops))
    vectors = (c_void_p * max(count, 1))(*(v for _, _, v in ops))
    entry = lib().krn_gemm_nt
    head = (kind(in_dtype), a, b, c, kind(out_dtype), m, n, k, count, codes, scalars, vectors)

    def call(stream: int) -> None:
        check(entry(*head, stream), "krn_gemm_nt")

    return call


def marshal_ops(ops: list[tuple[int, float, int]]):
    """The (codes, scalars, vectors) arrays of an epilogue chain for the GEMM entry points."""
    count = len(ops)
    return ((c_int * max(count, 1))(*(op for op, _, _ in ops)), (c_float * max(count, 1))(*(s for _, s, _ in ops)),
            (c_void_p * max(count, 1))(*(v for _, _, v in ops)))


def gemm_nn_workspace(n: int, k: int) -> int:
    """Bytes of device workspace krn_gemm_nn needs for a K x N operand B."""
    return lib().krn_gemm_nn_workspace(n, k)


def gemm_nn_workspace_for(a: int, b: int, m: int, n: int, k: int) -> int:
    """Bytes of workspace this NN product needs: 0 when the kernel reads B as it lies."""
    return lib().krn_gemm_nn_workspace_for(a, b, m, n, k)


def gemm_nn_call(in_dtype: Dtype, a: int, b: int, c: int, out_dtype: Dtype, m: int, n: int, k: int,
                 ops: list[tuple[int, float, int]], workspace: int, workspace_bytes: int):
    """`gemm_nn` (B stored K x N, read as it lies or transposed into `workspace`) as a function of the stream,
    marshalled once."""
    count = len(ops)
    codes = (c_int * max(count, 1))(*(op for op, _, _ in ops))
    scalars = (c_float * max(count, 1))(*(s for _, s, _ in ops))
    vectors = (c_void_p * max(count, 1))(*(v for _, _, v in ops))
    entry = lib().krn_gemm_nn
    head = (kind(in_dtype), a, b, c, kind(out_dtype), m, n, k, count, codes, scalars, vectors, workspace,
            workspace_bytes)

    def call(stream: int) -> None:
        check(entry(*head, stream), "krn_gemm_nn")

    return call


def gemm_nt(in_dtype: Dtype, a: int, b: int, c: int, out_dtype: Dtype, m: int, n: int, k: int,
            ops: list[tuple[int, float, int]], stream: int) -> None:
    """C[m, n] = epilogue(sum_k A[m, k] B[n, k]); `ops` are (operation, scalar, vector pointer)."""
    gemm_nt_call(in_dtype, a, b, c, out_dtype, m, n, k, ops)(stream)


def attention_fwd(dtype: Dtype, q: int, k: int, v: int, o: int, bh: int, sq: int, sk: int, d: int, scale: float,
                  causal: bool, stream: int) -> None:
    check(lib().krn_attention_fwd(kind(dtype), q, k, v, o, bh, sq, sk, d, scale, int(causal), stream),
          "krn_attention_fwd")


def transpose16(src: int, dst: int, rows: int, cols: int, stream: int) -> None:
    """dst (cols x rows) = src (rows x cols) transposed, 16-bit elements."""
    check(lib().krn_transpose16(src, dst, rows, cols, stream), "krn_transpose16")


def softmax_rows(dtype: Dtype, x: int, y: int, rows: int, width: int, ldx: int, ldy: int, stream: int) -> None:
    """y = softmax over the first `width` columns of each row of x (row strides ldx, ldy in elements)."""
    check(lib().krn_softmax_rows(kind(dtype), x, y, rows, width, ldx, ldy, stream), "krn_softmax_rows")

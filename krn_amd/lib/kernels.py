"""The multiply behind `lib.matmul`'s own candidate: one tiled tile program whose bias and activation are chosen by
constants (reference src/krn/lib/lib_kernels.py:20-48, `MatmulTiling` and `matmul_epilogue`).

The program is generic over its element type F, as the reference's is: `Matrix[F]` takes the element type of the
argument it is launched with. A constant that is False folds its branch away at capture, so each epilogue is its
own program. The accumulator is float32; the result is rounded once, to the type of `out`. On gfx950 a 16-bit
program lowers to the MFMA GEMM with the bias and activation fused into its epilogue, an f32 one to the generic
lowering.
"""

from typing import TypeVar

from krn_amd import Const, Matrix, T, Vector, block, kernel, pipelined, struct, zeros

F = TypeVar("F")


@struct
class MatmulTiling:
    bm: Const[int] = 16
    bn: Const[int] = 16
    bk: Const[int] = 8
    bias: Const[bool] = False
    relu: Const[bool] = False
    gelu: Const[bool] = False
    silu: Const[bool] = False


@kernel
def matmul_epilogue(t: MatmulTiling, a: Matrix[F], b: Matrix[F], bias: Vector[F], out: Matrix[F]) -> None:
    """`out = activation(a @ b + bias)`; `bias` is read only when `t.bias` is set."""
    rows, cols = block.tile(t.bm, t.bn)
    acc = zeros(T.f32, t.bm, t.bn)
    for ks in pipelined(a.shape[1], t.bk):
        acc += a[rows, ks] @ b[ks, cols]
    if t.bias:
        acc += bias[cols].to(T.f32)
    if t.relu:
        acc = acc.relu()
    if t.gelu:
        acc = acc.gelu()
    if t.silu:
        acc = acc.silu()
    out[rows, cols] = acc.to(out.dtype)

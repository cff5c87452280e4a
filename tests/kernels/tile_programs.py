"""krn tile programs the tests and the benchmark run unchanged on the CPU oracle and on gfx950.

`matmul` and `flash_attention` are krn's own example programs (reference examples/04_libraries/01_gemm_tiles.py:34-40
and 08_flash_attention.py:35-59), restated here because the kernels must be the same programs; `gemm_nt` is the
`C = A @ B^T` form of the benchmark configuration, and the quantized GEMMs add the scale epilogues. The small tile
kernels mirror the operations of reference tests/kernels/tile_ops.py. `matmul_epilogue` is the kernel behind krn's
`lib.matmul` (reference src/krn/lib/lib_kernels.py:20-48); the reference declares it generic over F with Python
3.12 syntax, so it is stated here once per dtype it runs with (f16 and f32).
"""

from krn_amd import Const, Matrix, T, Tensor, Vector, arange, block, kernel, maximum, pipelined, struct, where, zeros


@struct
class Tiling:
    bm: Const[int] = 128
    bn: Const[int] = 128
    bk: Const[int] = 32


@kernel
def matmul(t: Tiling, a: Matrix[T.f16], b: Matrix[T.f16], c: Matrix[T.f16]) -> None:
    rows, cols = block.tile(t.bm, t.bn)
    acc = zeros(T.f32, t.bm, t.bn)
    for ks in pipelined(a.shape[1], t.bk):
        acc += a[rows, ks] @ b[ks, cols]
    c[rows, cols] = acc.to(T.f16)


@kernel
def gemm_nt(t: Tiling, a: Matrix[T.bf16], b: Matrix[T.bf16], c: Matrix[T.bf16]) -> None:
    rows, cols = block.tile(t.bm, t.bn)
    acc = zeros(T.f32, t.bm, t.bn)
    for ks in pipelined(a.shape[1], t.bk):
        acc += a[rows, ks] @ b[cols, ks].transpose()
    c[rows, cols] = acc.to(T.bf16)


@kernel
def gemm_nt_f32(t: Tiling, a: Matrix[T.bf16], b: Matrix[T.bf16], c: Matrix[T.f32]) -> None:
    rows, cols = block.tile(t.bm, t.bn)
    acc = zeros(T.f32, t.bm, t.bn)
    for ks in pipelined(a.shape[1], t.bk):
        acc += a[rows, ks] @ b[cols, ks].transpose()
    c[rows, cols] = acc


@kernel
def gemm_fp8(
    t: Tiling, a: Matrix[T.f8e4m3fn], b: Matrix[T.f8e4m3fn], c: Matrix[T.bf16], scale_a: T.f32, scale_b: T.f32
) -> None:
    rows, cols = block.tile(t.bm, t.bn)
    acc = zeros(T.f32, t.bm, t.bn)
    for ks in pipelined(a.shape[1], t.bk):
        acc += a[rows, ks] @ b[cols, ks].transpose()
    c[rows, cols] = (acc * (scale_a * scale_b)).to(T.bf16)


@kernel
def gemm_w8a8(
    t: Tiling,
    a: Matrix[T.i8],
    w: Matrix[T.i8],
    scale_a: Matrix[T.f32],
    scale_w: Matrix[T.f32],
    c: Matrix[T.bf16],
) -> None:
    rows, cols = block.tile(t.bm, t.bn)
    acc = zeros(T.i32, t.bm, t.bn)
    for ks in pipelined(a.shape[1], t.bk):
        acc += a[rows, ks] @ w[cols, ks].transpose()
    c[rows, cols] = (acc.to(T.f32) * scale_a[rows, 0:1] * scale_w[0:1, cols]).to(T.bf16)


@kernel
def gemm_i8_i32(t: Tiling, a: Matrix[T.i8], w: Matrix[T.i8], c: Matrix[T.i32]) -> None:
    rows, cols = block.tile(t.bm, t.bn)
    acc = zeros(T.i32, t.bm, t.bn)
    for ks in pipelined(a.shape[1], t.bk):
        acc += a[rows, ks] @ w[cols, ks].transpose()
    c[rows, cols] = acc


@struct
class Attention:
    bq: Const[int] = 16
    bk: Const[int] = 16
    d: Const[int] = 64
    causal: Const[bool] = False


@kernel
def flash_attention(
    t: Attention,
    q: Tensor[T.f16, int, int, int],
    k: Tensor[T.f16, int, int, int],
    v: Tensor[T.f16, int, int, int],
    o: Tensor[T.f16, int, int, int],
    scale: T.f32,
) -> None:
    rows, head = block.tile(t.bq), block.index().y
    q_pos = arange(t.bq, 0, rank=2, start=block.index().x * t.bq)
    m, total, acc = zeros(T.f32, t.bq, 1).sub(1.0e30), zeros(T.f32, t.bq, 1), zeros(T.f32, t.bq, t.d)
    qt = q[head, rows, slice(0, t.d)]
    for c in range(0, k.shape[1], t.bk):
        s = (qt @ k[head, c : c + t.bk, slice(0, t.d)].transpose()).mul(scale)
        if t.causal:
            s = where(arange(t.bk, 1, rank=2, start=c) <= q_pos, s, -1.0e30)
        m_new = m.maximum(s.max(keepdims=True))
        p, corr = (s - m_new).exp2(), (m - m_new).exp2()
        total *= corr
        total += p.sum(keepdims=True)
        acc *= corr
        acc += p.to(T.f16) @ v[head, c : c + t.bk, slice(0, t.d)]
        m = m_new
    o[head, rows, slice(0, t.d)] = (acc / total).to(T.f16)


@kernel
def flash_attention_bf16(
    t: Attention,
    q: Tensor[T.bf16, int, int, int],
    k: Tensor[T.bf16, int, int, int],
    v: Tensor[T.bf16, int, int, int],
    o: Tensor[T.bf16, int, int, int],
    scale: T.f32,
) -> None:
    rows, head = block.tile(t.bq), block.index().y
    q_pos = arange(t.bq, 0, rank=2, start=block.index().x * t.bq)
    m, total, acc = zeros(T.f32, t.bq, 1).sub(1.0e30), zeros(T.f32, t.bq, 1), zeros(T.f32, t.bq, t.d)
    qt = q[head, rows, slice(0, t.d)]
    for c in range(0, k.shape[1], t.bk):
        s = (qt @ k[head, c : c + t.bk, slice(0, t.d)].transpose()).mul(scale)
        if t.causal:
            s = where(arange(t.bk, 1, rank=2, start=c) <= q_pos, s, -1.0e30)
        m_new = m.maximum(s.max(keepdims=True))
        p, corr = (s - m_new).exp2(), (m - m_new).exp2()
        total *= corr
        total += p.sum(keepdims=True)
        acc *= corr
        acc += p.to(T.bf16) @ v[head, c : c + t.bk, slice(0, t.d)]
        m = m_new
    o[head, rows, slice(0, t.d)] = (acc / total).to(T.bf16)


@struct
class Shape:
    rows: Const[int] = 8
    cols: Const[int] = 16


@kernel
def transpose(t: Shape, x: Matrix[T.f32], y: Matrix[T.f32]) -> None:
    y[0 : t.cols, 0 : t.rows] = x[0 : t.rows, 0 : t.cols].transpose()


@kernel
def select(t: Shape, x: Matrix[T.f32], y: Matrix[T.f32]) -> None:
    tile = x[0 : t.rows, 0 : t.cols]
    y[0 : t.rows, 0 : t.cols] = where(tile > 0.0, tile, 0.5)


@kernel
def compare(
    t: Shape,
    x: Matrix[T.f32],
    less: Matrix[T.f32],
    less_equal: Matrix[T.f32],
    greater: Matrix[T.f32],
    greater_equal: Matrix[T.f32],
) -> None:
    tile = x[0 : t.rows, 0 : t.cols]
    less[0 : t.rows, 0 : t.cols] = (tile < 0.0).to(T.f32)
    less_equal[0 : t.rows, 0 : t.cols] = (tile <= 0.0).to(T.f32)
    greater[0 : t.rows, 0 : t.cols] = (tile > 0.0).to(T.f32)
    greater_equal[0 : t.rows, 0 : t.cols] = (tile >= 0.0).to(T.f32)


@kernel
def positions(t: Shape, out: Matrix[T.i32]) -> None:
    rows = arange(t.rows, 0, rank=2, start=3)
    cols = arange(t.cols, 1, rank=2)
    out[0 : t.rows, 0 : t.cols] = cols - rows


@kernel
def product(t: Shape, x: Matrix[T.f16], w: Matrix[T.f16], y: Matrix[T.f32]) -> None:
    y[0 : t.rows, 0 : t.rows] = x[0 : t.rows, 0 : t.cols] @ w[0 : t.rows, 0 : t.cols].transpose()


@kernel
def per_head(t: Shape, x: Tensor[T.f32, int, int, int], y: Tensor[T.f32, int, int, int]) -> None:
    head = block.index().y
    y[head, 0 : t.rows, 0 : t.cols] = x[head, 0 : t.rows, 0 : t.cols] * 2.0


@kernel
def causal(t: Shape, x: Matrix[T.f32], y: Matrix[T.f32]) -> None:
    rows = arange(t.rows, 0, rank=2)
    cols = arange(t.cols, 1, rank=2)
    y[0 : t.rows, 0 : t.cols] = where(cols <= rows, x[0 : t.rows, 0 : t.cols], -1.0e30)


@kernel
def scaled_by_extent(t: Shape, x: Matrix[T.f32], y: Matrix[T.f32]) -> None:
    tile = x[0 : t.rows, 0 : t.cols]
    y[0 : t.rows, 0 : t.cols] = tile * tile.shape[1]


@kernel
def row_softmax(t: Shape, x: Matrix[T.f32], y: Matrix[T.f32]) -> None:
    rows = block.tile(t.rows)
    tile = x[0 : t.rows, 0 : t.cols]
    shifted = (tile - tile.max(axis=1, keepdims=True)).exp()
    y[0 : t.rows, 0 : t.cols] = shifted / shifted.sum(axis=1, keepdims=True)


@kernel
def matmul_f32(t: Tiling, a: Matrix[T.f32], b: Matrix[T.f32], c: Matrix[T.f32]) -> None:
    rows, cols = block.tile(t.bm, t.bn)
    acc = zeros(T.f32, t.bm, t.bn)
    for ks in pipelined(a.shape[1], t.bk):
        acc += a[rows, ks] @ b[ks, cols]
    c[rows, cols] = acc


@kernel
def matmul_f16_f32(t: Tiling, a: Matrix[T.f16], b: Matrix[T.f16], c: Matrix[T.f32]) -> None:
    rows, cols = block.tile(t.bm, t.bn)
    acc = zeros(T.f32, t.bm, t.bn)
    for ks in pipelined(a.shape[1], t.bk):
        acc += a[rows, ks] @ b[ks, cols]
    c[rows, cols] = acc


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
def matmul_epilogue(
    t: MatmulTiling, a: Matrix[T.f16], b: Matrix[T.f16], bias: Vector[T.f16], out: Matrix[T.f16]
) -> None:
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


@kernel
def matmul_epilogue_f32(
    t: MatmulTiling, a: Matrix[T.f32], b: Matrix[T.f32], bias: Vector[T.f32], out: Matrix[T.f32]
) -> None:
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


# krn's softmax programs (reference examples/02_tiles_and_types/01_softmax_rows.py:27-40 and
# tests/helpers/example_softmax.py:12-24), unchanged


@struct
class RowTiling:
    rows: Const[int] = 4
    cols: Const[int] = 1024


@kernel
def softmax_long_rows(t: RowTiling, x: Matrix[T.f16], y: Matrix[T.f16]) -> None:
    rows = block.tile(t.rows)
    m = zeros(T.f32, t.rows, 1).sub(3.0e38)  # a finite stand-in for -inf, which a kernel cannot spell yet
    s = zeros(T.f32, t.rows, 1)
    for cs in pipelined(x.shape[1], t.cols):  # column chunks, the last one ragged
        v = x[rows, cs].to(T.f32)
        m_new = maximum(m, v.max(keepdims=True))
        s = s * (m - m_new).exp() + (v - m_new).exp().sum(keepdims=True)
        m = m_new
    for cs in pipelined(x.shape[1], t.cols):
        y[rows, cs] = (x[rows, cs].to(T.f32) - m).exp().div(s).to(T.f16)


@kernel
def softmax(x: Matrix[T.f16], y: Matrix[T.f16], t: RowTiling) -> None:
    rows, cols = block.tile(t.rows), slice(0, t.cols)
    y[rows, cols] = x[rows, cols].to(T.f32).softmax(axis=1).to(T.f16)


@kernel
def softmax_steps(x: Matrix[T.f16], y: Matrix[T.f16], t: RowTiling) -> None:
    """The same function with its arithmetic spelled out: subtract the row maximum, exponentiate, normalize."""
    rows, cols = block.tile(t.rows), slice(0, t.cols)
    v = x[rows, cols].to(T.f32)
    e = (v - v.max(axis=1, keepdims=True)).exp()
    y[rows, cols] = (e / e.sum(axis=1, keepdims=True)).to(T.f16)


# the same programs written for bf16 and f32 tensors


@kernel
def softmax_long_rows_bf16(t: RowTiling, x: Matrix[T.bf16], y: Matrix[T.bf16]) -> None:
    rows = block.tile(t.rows)
    m = zeros(T.f32, t.rows, 1).sub(3.0e38)
    s = zeros(T.f32, t.rows, 1)
    for cs in pipelined(x.shape[1], t.cols):
        v = x[rows, cs].to(T.f32)
        m_new = maximum(m, v.max(keepdims=True))
        s = s * (m - m_new).exp() + (v - m_new).exp().sum(keepdims=True)
        m = m_new
    for cs in pipelined(x.shape[1], t.cols):
        y[rows, cs] = (x[rows, cs].to(T.f32) - m).exp().div(s).to(T.bf16)


@kernel
def softmax_bf16(x: Matrix[T.bf16], y: Matrix[T.bf16], t: RowTiling) -> None:
    rows, cols = block.tile(t.rows), slice(0, t.cols)
    y[rows, cols] = x[rows, cols].to(T.f32).softmax(axis=1).to(T.bf16)


@kernel
def softmax_f32(x: Matrix[T.f32], y: Matrix[T.f32], t: RowTiling) -> None:
    rows, cols = block.tile(t.rows), slice(0, t.cols)
    y[rows, cols] = x[rows, cols].to(T.f32).softmax(axis=1).to(T.f32)


@struct
class PartialK:
    bm: Const[int] = 64
    bn: Const[int] = 64
    bk: Const[int] = 32
    kk: Const[int] = 96


@kernel
def gemm_partial_k(t: PartialK, a: Matrix[T.bf16], b: Matrix[T.bf16], c: Matrix[T.f32]) -> None:
    """The product over the first t.kk columns of K only: not the whole product, so the generic lowering runs it,
    its products on the matrix cores."""
    rows, cols = block.tile(t.bm, t.bn)
    acc = zeros(T.f32, t.bm, t.bn)
    for ks in pipelined(t.kk, t.bk):
        acc += a[rows, ks] @ b[cols, ks].transpose()
    c[rows, cols] = acc


@kernel
def gemm_i8_partial_k(t: PartialK, a: Matrix[T.i8], b: Matrix[T.i8], c: Matrix[T.i32]) -> None:
    rows, cols = block.tile(t.bm, t.bn)
    acc = zeros(T.i32, t.bm, t.bn)
    for ks in pipelined(t.kk, t.bk):
        acc += a[rows, ks] @ b[cols, ks].transpose()
    c[rows, cols] = acc

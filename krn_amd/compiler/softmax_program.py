"""krn's row-softmax tile programs, the ones the gfx950 row-softmax kernel implements.

The programs are krn's own: the long-row form with a running maximum and sum over column chunks (reference
examples/02_tiles_and_types/01_softmax_rows.py:27-40) and the one-tile forms, `.softmax(axis=1)` and its spelled-out
steps (reference tests/helpers/example_softmax.py:12-24). They are written out here because `cdna4.match_softmax`
recognises a user's kernel by comparing its captured IR with these. The tensors may be f16, bf16 or f32 (capture
overrides the annotations; the casts follow the tensors).
"""

from krn_amd import Const, T, Tensor, block, kernel, maximum, pipelined, struct, zeros


@struct
class RowTiling:
    rows: Const[int] = 4
    cols: Const[int] = 1024


@kernel
def softmax_long_rows(t: RowTiling, x: Tensor[T.f16, int, int], y: Tensor[T.f16, int, int]) -> None:
    rows = block.tile(t.rows)
    m = zeros(T.f32, t.rows, 1).sub(3.0e38)
    s = zeros(T.f32, t.rows, 1)
    for cs in pipelined(x.shape[1], t.cols):
        v = x[rows, cs].to(T.f32)
        m_new = maximum(m, v.max(keepdims=True))
        s = s * (m - m_new).exp() + (v - m_new).exp().sum(keepdims=True)
        m = m_new
    for cs in pipelined(x.shape[1], t.cols):
        y[rows, cs] = (x[rows, cs].to(T.f32) - m).exp().div(s).to(T.f16)


@kernel
def softmax(x: Tensor[T.f16, int, int], y: Tensor[T.f16, int, int], t: RowTiling) -> None:
    rows, cols = block.tile(t.rows), slice(0, t.cols)
    y[rows, cols] = x[rows, cols].to(T.f32).softmax(axis=1).to(T.f16)


@kernel
def softmax_steps(x: Tensor[T.f16, int, int], y: Tensor[T.f16, int, int], t: RowTiling) -> None:
    rows, cols = block.tile(t.rows), slice(0, t.cols)
    v = x[rows, cols].to(T.f32)
    e = (v - v.max(axis=1, keepdims=True)).exp()
    y[rows, cols] = (e / e.sum(axis=1, keepdims=True)).to(T.f16)

"""krn's flash-attention tile program, the one the gfx950 attention kernel implements.

The program is krn's own example (reference examples/04_libraries/08_flash_attention.py:35-59); it is written out
here because `cdna4.match_attention` recognises a user's kernel by comparing its captured IR with this one's. The
parameters may be f16 or bf16 (capture overrides the annotations).
"""

from krn_amd import Const, T, Tensor, arange, block, kernel, struct, where, zeros


@struct
class Tiling:
    bq: Const[int] = 16
    bk: Const[int] = 16
    d: Const[int] = 64
    causal: Const[bool] = False


@kernel
def flash_attention(
    t: Tiling,
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

"""Flash-attention tile programs written differently from krn's example (reference
examples/04_libraries/08_flash_attention.py:35-59) but computing the same online softmax: the gfx950 lowering must
recognise them by what they compute and run them on the hand-written attention kernel. `drifting` and
`unscaled_sum` differ in what they compute and must not be recognised."""

from krn_amd import Const, T, Tensor, arange, block, kernel, maximum, struct, where, zeros


@struct
class Shape:
    rows_per_block: Const[int] = 256
    keys_per_step: Const[int] = 32
    head_dim: Const[int] = 128
    masked: Const[bool] = True


@kernel
def reordered(
    cfg: Shape,
    query: Tensor[T.bf16, int, int, int],
    key: Tensor[T.bf16, int, int, int],
    value: Tensor[T.bf16, int, int, int],
    out: Tensor[T.bf16, int, int, int],
    softmax_scale: T.f32,
) -> None:
    """Other names and tiling, `scale * s` on the left, the mask as `q_pos >= k_pos`, `maximum(...)` as a function,
    temporaries for the row statistics and the updates written as plain assignments."""
    rows = block.tile(cfg.rows_per_block)
    h = block.index().y
    first_row = block.index().x * cfg.rows_per_block
    q_tile = query[h, rows, slice(0, cfg.head_dim)]
    running_max = zeros(T.f32, cfg.rows_per_block, 1) - 1.0e30
    denominator = zeros(T.f32, cfg.rows_per_block, 1)
    numerator = zeros(T.f32, cfg.rows_per_block, cfg.head_dim)
    for start in range(0, key.shape[1], cfg.keys_per_step):
        raw = q_tile @ key[h, start : start + cfg.keys_per_step, slice(0, cfg.head_dim)].transpose()
        scores = softmax_scale * raw
        if cfg.masked:
            query_pos = arange(cfg.rows_per_block, 0, rank=2, start=first_row)
            key_pos = arange(cfg.keys_per_step, 1, rank=2, start=start)
            scores = where(query_pos >= key_pos, scores, -1.0e30)
        tile_max = scores.max(keepdims=True)
        new_max = maximum(tile_max, running_max)
        rescale = (running_max - new_max).exp2()
        weights = (scores - new_max).exp2()
        tile_sum = weights.sum(keepdims=True)
        denominator = tile_sum + denominator * rescale
        numerator = rescale * numerator
        numerator += weights.to(T.bf16) @ value[h, start : start + cfg.keys_per_step, slice(0, cfg.head_dim)]
        running_max = new_max
    out[h, rows, slice(0, cfg.head_dim)] = (numerator / denominator).to(T.bf16)


@struct
class Natural:
    bq: Const[int] = 128
    bk: Const[int] = 64
    d: Const[int] = 128
    causal: Const[bool] = True


@kernel
def natural_exp_4d(
    t: Natural,
    q: Tensor[T.bf16, int, int, int, int],
    k: Tensor[T.bf16, int, int, int, int],
    v: Tensor[T.bf16, int, int, int, int],
    o: Tensor[T.bf16, int, int, int, int],
    scale: T.f32,
) -> None:
    """(batch, heads, seq, d) tensors indexed by blocks z and y, the natural exponential, the scale applied to the
    product by `.mul`, and the mask written as `k_pos > q_pos` with the branches swapped."""
    rows = block.tile(t.bq)
    b, h = block.index().z, block.index().y
    q_pos = arange(t.bq, 0, rank=2, start=block.index().x * t.bq)
    m = zeros(T.f32, t.bq, 1) - 1.0e30
    total = zeros(T.f32, t.bq, 1)
    acc = zeros(T.f32, t.bq, t.d)
    for c in range(0, k.shape[2], t.bk):
        s = (q[b, h, rows, slice(0, t.d)] @ k[b, h, c : c + t.bk, slice(0, t.d)].transpose()).mul(scale)
        if t.causal:
            s = where(arange(t.bk, 1, rank=2, start=c) > q_pos, -1.0e30, s)
        m_new = m.maximum(s.max(keepdims=True))
        p, corr = (s - m_new).exp(), (m - m_new).exp()
        total = total * corr + p.sum(keepdims=True)
        acc = acc * corr
        acc += p.to(T.bf16) @ v[b, h, c : c + t.bk, slice(0, t.d)]
        m = m_new
    o[b, h, rows, slice(0, t.d)] = (acc / total).to(T.bf16)


@kernel
def drifting(
    t: Natural,
    q: Tensor[T.bf16, int, int, int],
    k: Tensor[T.bf16, int, int, int],
    v: Tensor[T.bf16, int, int, int],
    o: Tensor[T.bf16, int, int, int],
    scale: T.f32,
) -> None:
    """Not attention: the output is not rescaled when the running maximum moves."""
    rows, head = block.tile(t.bq), block.index().y
    m, total, acc = zeros(T.f32, t.bq, 1) - 1.0e30, zeros(T.f32, t.bq, 1), zeros(T.f32, t.bq, t.d)
    qt = q[head, rows, slice(0, t.d)]
    for c in range(0, k.shape[1], t.bk):
        s = (qt @ k[head, c : c + t.bk, slice(0, t.d)].transpose()).mul(scale)
        m_new = m.maximum(s.max(keepdims=True))
        p, corr = (s - m_new).exp2(), (m - m_new).exp2()
        total = total * corr + p.sum(keepdims=True)
        acc += p.to(T.bf16) @ v[head, c : c + t.bk, slice(0, t.d)]
        m = m_new
    o[head, rows, slice(0, t.d)] = (acc / total).to(T.bf16)


@kernel
def unscaled_sum(
    t: Natural,
    q: Tensor[T.bf16, int, int, int],
    k: Tensor[T.bf16, int, int, int],
    v: Tensor[T.bf16, int, int, int],
    o: Tensor[T.bf16, int, int, int],
    scale: T.f32,
) -> None:
    """Not attention: the row sum mixes the natural exponential into an exp2 softmax."""
    rows, head = block.tile(t.bq), block.index().y
    m, total, acc = zeros(T.f32, t.bq, 1) - 1.0e30, zeros(T.f32, t.bq, 1), zeros(T.f32, t.bq, t.d)
    qt = q[head, rows, slice(0, t.d)]
    for c in range(0, k.shape[1], t.bk):
        s = (qt @ k[head, c : c + t.bk, slice(0, t.d)].transpose()).mul(scale)
        m_new = m.maximum(s.max(keepdims=True))
        p, corr = (s - m_new).exp2(), (m - m_new).exp()
        total = total * corr + p.sum(keepdims=True)
        acc = acc * corr
        acc += p.to(T.bf16) @ v[head, c : c + t.bk, slice(0, t.d)]
        m = m_new
    o[head, rows, slice(0, t.d)] = (acc / total).to(T.bf16)

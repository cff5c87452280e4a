"""Row-softmax tile programs written differently from krn's (reference examples/02_tiles_and_types/
01_softmax_rows.py:27-40, tests/helpers/example_softmax.py:12-24) that compute the same thing, and two that do not
(`unshifted`: no maximum subtracted; `reciprocal`: a multiply by 1 / sum, another rounding)."""

from krn_amd import Const, T, Tensor, block, kernel, maximum, pipelined, struct, zeros


@struct
class Rows:
    per_block: Const[int] = 2
    chunk: Const[int] = 256


@kernel
def running(cfg: Rows, src: Tensor[T.f16, int, int], dst: Tensor[T.f16, int, int]) -> None:
    """The long-row form with other names, `maximum(rowmax, m)` in the other order, the sum update written the
    other way round, and temporaries."""
    r = block.tile(cfg.per_block)
    best = zeros(T.f32, cfg.per_block, 1) - 3.0e38
    norm = zeros(T.f32, cfg.per_block, 1)
    for part in pipelined(src.shape[1], cfg.chunk):
        vals = src[r, part].to(T.f32)
        top = maximum(vals.max(keepdims=True), best)
        shift = (best - top).exp()
        norm = (vals - top).exp().sum(keepdims=True) + norm * shift
        best = top
    for part in pipelined(src.shape[1], cfg.chunk):
        vals = src[r, part].to(T.f32)
        dst[r, part] = ((vals - best).exp() / norm).to(T.f16)


@struct
class Tile:
    per_block: Const[int] = 4
    width: Const[int] = 96


@kernel
def one_tile(cfg: Tile, src: Tensor[T.f16, int, int], dst: Tensor[T.f16, int, int]) -> None:
    r = block.tile(cfg.per_block)
    vals = src[r, slice(0, cfg.width)].to(T.f32)
    peak = vals.max(axis=1, keepdims=True)
    w = (vals - peak).exp()
    total = w.sum(axis=1, keepdims=True)
    dst[r, slice(0, cfg.width)] = (w / total).to(T.f16)


@kernel
def unshifted(cfg: Tile, src: Tensor[T.f16, int, int], dst: Tensor[T.f16, int, int]) -> None:
    r = block.tile(cfg.per_block)
    w = src[r, slice(0, cfg.width)].to(T.f32).exp()
    dst[r, slice(0, cfg.width)] = (w / w.sum(axis=1, keepdims=True)).to(T.f16)


@kernel
def reciprocal(cfg: Tile, src: Tensor[T.f16, int, int], dst: Tensor[T.f16, int, int]) -> None:
    r = block.tile(cfg.per_block)
    vals = src[r, slice(0, cfg.width)].to(T.f32)
    w = (vals - vals.max(axis=1, keepdims=True)).exp()
    dst[r, slice(0, cfg.width)] = (w * (1.0 / w.sum(axis=1, keepdims=True))).to(T.f16)

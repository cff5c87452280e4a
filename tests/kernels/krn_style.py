"""Stand-ins shaped like krn's own host objects, for launching through this backend the way krn itself would.

- `Kernel` carries only `fn` and `name` (and a lazily filled `_shape`), as reference src/krn/frontend/kernel.py:38-40
  does: no parameter table, no configuration accessor.
- `Const` is a generic alias whose origin is named `Const`, as krn's `type Const[T] = T` (reference
  src/krn/frontend/records.py:17) is under `typing.get_origin`.
- `fp`, `sint` and `uint` are parametrised element-type families, subscripted with literal widths and a format kind
  class (reference src/krn/frontend/numerics.py:343-384: `bf16 = fp[L[8], L[7], ieee]`).
- `Blocks` and `Tiles` have the public fields of reference src/krn/frontend/geometry.py:15-39.

`gemm_nt` and `flash_attention` are krn tile programs written against those objects; their bodies use the tile
vocabulary this backend captures from source.
"""

from dataclasses import dataclass
from typing import Generic, Literal as L, TypeVar

from krn_amd import Matrix, T, Tensor, arange, block, pipelined, where, zeros

V = TypeVar("V")
E = TypeVar("E")
M = TypeVar("M")


class Const(Generic[V]):
    pass


class ieee:
    pass


class fn:
    pass


class fp(Generic[E, M, V]):
    pass


class sint(Generic[V]):
    pass


class uint(Generic[V]):
    pass


bf16 = fp[L[8], L[7], ieee]
f16 = fp[L[5], L[10], ieee]
f32 = fp[L[8], L[23], ieee]
f8e4m3fn = fp[L[4], L[3], fn]
i8 = sint[L[8]]
i32 = sint[L[32]]


def struct(cls):
    return dataclass(frozen=True)(cls)


@dataclass(frozen=True)
class Blocks:
    x: int
    y: int = 1
    z: int = 1
    threads: int | None = None


@dataclass(frozen=True)
class Tiles:
    shape: tuple[int, ...]
    tile: tuple[int, ...]

    @property
    def blocks(self) -> Blocks:
        counts = [-(-extent // size) for extent, size in zip(self.shape, self.tile, strict=True)]
        return Blocks(*reversed(counts))


class Kernel:
    __slots__ = ("_shape", "fn", "name")

    def __init__(self, fn) -> None:
        self.fn = fn
        self.name = getattr(fn, "__name__", type(fn).__name__)
        self._shape = None


def kernel(fn) -> Kernel:
    return Kernel(fn)


@struct
class Tiling:
    bm: Const[int] = 256
    bn: Const[int] = 256
    bk: Const[int] = 64


@kernel
def gemm_nt(t: Tiling, a: Matrix[T.bf16], b: Matrix[T.bf16], c: Matrix[T.bf16]) -> None:
    rows, cols = block.tile(t.bm, t.bn)
    acc = zeros(T.f32, t.bm, t.bn)
    for ks in pipelined(a.shape[1], t.bk):
        acc += a[rows, ks] @ b[cols, ks].transpose()
    c[rows, cols] = acc.to(T.bf16)


@struct
class Attention:
    bq: Const[int] = 128
    bk: Const[int] = 64
    d: Const[int] = 128
    causal: Const[bool] = True


@kernel
def flash_attention(
    t: Attention,
    q: Tensor[T.bf16, int, int, int],
    k: Tensor[T.bf16, int, int, int],
    v: Tensor[T.bf16, int, int, int],
    o: Tensor[T.bf16, int, int, int],
    scale: T.f32,
) -> None:
    """krn's flash-attention example (reference examples/04_libraries/08_flash_attention.py:35-59) with bf16 tiles."""
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

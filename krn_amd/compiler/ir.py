"""The typed IR of a captured tile kernel: structured statements over typed expressions.

The node set follows krn's IR (reference src/krn/compiler/ir.py:16-452) for the subset the tile path uses: scalar
and tile values, tile loads/stores with invalid lanes, `Accumulate` (`acc += lhs @ rhs` with float32 products and
sums, or int32 for int8 operands), `Transpose`, `Arange`, `Select`, `Reduce`, elementwise `Math`, `Cast`, and
`For` loops (pipelined or not). Every tile extent is a capture-time constant.
"""

from dataclasses import dataclass, field
from enum import Enum

from krn_amd.dtypes import I64, PY_INT, Dtype


class Op(Enum):
    ADD = "+"
    SUB = "-"
    MUL = "*"
    DIV = "/"
    MOD = "%"
    LT = "<"
    LE = "<="
    GT = ">"
    GE = ">="
    EQ = "=="
    NE = "!="
    AND = "&"
    OR = "|"
    NEG = "neg"


COMPARISONS = (Op.LT, Op.LE, Op.GT, Op.GE, Op.EQ, Op.NE)


class Fn(Enum):
    EXP = "exp"
    EXP2 = "exp2"
    LOG = "log"
    LOG2 = "log2"
    SQRT = "sqrt"
    RSQRT = "rsqrt"
    ABS = "abs"
    TANH = "tanh"
    RELU = "relu"
    GELU = "gelu"
    SILU = "silu"
    SIGMOID = "sigmoid"
    ERF = "erf"
    MAXIMUM = "maximum"
    MINIMUM = "minimum"


class Reduction(Enum):
    MAX = "max"
    MIN = "min"
    SUM = "sum"


@dataclass(frozen=True)
class TileType:
    dtype: Dtype
    shape: tuple[int, ...]


@dataclass(frozen=True)
class SliceType:
    extent: int


@dataclass(frozen=True)
class TensorType:
    """A row-major view of global memory; its shape travels with the pointer (one i64 extent per axis)."""

    dtype: Dtype
    rank: int


ValueType = Dtype | TileType | SliceType


@dataclass(frozen=True)
class TensorRef:
    name: str
    type: TensorType

    def dim(self, axis: int) -> str:
        return f"{self.name}_n{axis}"


@dataclass(frozen=True)
class Expr:
    type: ValueType
    line: int = field(default=0, kw_only=True, compare=False, repr=False)

    @property
    def dtype(self) -> Dtype:
        t = self.type
        if isinstance(t, TileType):
            return t.dtype
        if isinstance(t, SliceType):
            return PY_INT
        return t

    @property
    def shape(self) -> tuple[int, ...]:
        return self.type.shape if isinstance(self.type, TileType) else ()


@dataclass(frozen=True)
class Const(Expr):
    value: int | float | bool


@dataclass(frozen=True)
class Var(Expr):
    """A scalar local or a tile variable (its type says which)."""

    name: str


@dataclass(frozen=True)
class Param(Expr):
    """A scalar kernel parameter."""

    name: str


@dataclass(frozen=True)
class Dim(Expr):
    """`tensor.shape[axis]`, a runtime extent."""

    tensor: TensorRef
    axis: int


@dataclass(frozen=True)
class BlockIndex(Expr):
    """`block.index().x/y/z`."""

    axis: str


@dataclass(frozen=True)
class Unary(Expr):
    op: Op
    operand: Expr


@dataclass(frozen=True)
class Binary(Expr):
    op: Op
    lhs: Expr
    rhs: Expr


@dataclass(frozen=True)
class Math(Expr):
    fn: Fn
    args: tuple[Expr, ...]


@dataclass(frozen=True)
class Cast(Expr):
    operand: Expr


@dataclass(frozen=True)
class Select(Expr):
    cond: Expr
    then: Expr
    orelse: Expr


@dataclass(frozen=True)
class Transpose(Expr):
    operand: Expr


@dataclass(frozen=True)
class Arange(Expr):
    axis: int
    start: Expr


@dataclass(frozen=True)
class SliceExpr(Expr):
    """The half-open range [start, start + extent) of one tensor axis; a squeezed axis is a scalar index."""

    start: Expr
    squeeze: bool = False

    @property
    def extent(self) -> int:
        return self.type.extent if isinstance(self.type, SliceType) else 1


@dataclass(frozen=True)
class TileLoad(Expr):
    """A tile read; elements outside the tensor read as zero and are invalid lanes."""

    tensor: TensorRef
    slices: tuple[SliceExpr, ...]


@dataclass(frozen=True)
class Zeros(Expr):
    pass


@dataclass(frozen=True)
class Reduce(Expr):
    op: Reduction
    operand: Expr
    axis: int
    keepdims: bool


@dataclass(frozen=True)
class Stmt:
    line: int = field(default=0, kw_only=True, compare=False, repr=False)


@dataclass(frozen=True)
class Assign(Stmt):
    var: Var
    value: Expr


@dataclass(frozen=True)
class TileAssign(Stmt):
    var: Var
    value: Expr


@dataclass(frozen=True)
class TileStore(Stmt):
    tensor: TensorRef
    slices: tuple[SliceExpr, ...]
    value: Expr


@dataclass(frozen=True)
class Accumulate(Stmt):
    """acc += lhs @ rhs: float32 products and sums (int32 for int8 operands), one fused step per k in k order."""

    acc: Var
    lhs: Expr
    rhs: Expr


@dataclass(frozen=True)
class For(Stmt):
    var: Var
    lo: Expr
    hi: Expr
    step: int
    body: tuple[Stmt, ...]
    pipelined: bool = False
    stages: int = 0


@dataclass(frozen=True)
class If(Stmt):
    cond: Expr
    then: tuple[Stmt, ...]
    orelse: tuple[Stmt, ...]


@dataclass(frozen=True)
class Kernel:
    name: str
    params: tuple[tuple[str, Dtype | TensorType], ...]  # runtime parameters in order (Const struct fields folded)
    tiles: tuple[Var, ...]
    body: tuple[Stmt, ...]
    space: tuple[tuple[str, int, tuple[Expr, ...]], ...]  # (grid axis, tile size, extents) read from block.tile
    consts: tuple[tuple[str, tuple[tuple[str, object], ...]], ...] = ()
    source: str = ""
    signature: tuple[str, ...] = ()  # every parameter name in order, configurations included

    def tensor(self, name: str) -> TensorRef:
        for n, t in self.params:
            if n == name and isinstance(t, TensorType):
                return TensorRef(n, t)
        raise KeyError(name)


def tile_shape(slices: tuple[SliceExpr, ...]) -> tuple[int, ...]:
    return tuple(s.extent for s in slices if not s.squeeze)


def slots(name: str, kind: Dtype | TensorType) -> list[tuple[str, Dtype, str]]:
    """The flat C-level fields of one parameter: a tensor is a pointer plus one i64 extent per axis
    (reference src/krn/compiler/ir.py:441-452)."""
    if isinstance(kind, TensorType):
        return [(name, kind.dtype, "ptr"), *((f"{name}_n{a}", I64, "dim") for a in range(kind.rank))]
    return [(name, kind, "scalar")]


def children(e: Expr) -> tuple[Expr, ...]:
    match e:
        case Unary(operand=o) | Cast(operand=o) | Transpose(operand=o) | Reduce(operand=o):
            return (o,)
        case Binary(lhs=a, rhs=b):
            return (a, b)
        case Math(args=args):
            return args
        case Select(cond=c, then=t, orelse=o):
            return (c, t, o)
        case Arange(start=s):
            return (s,)
        case TileLoad(slices=slices):
            return slices
        case SliceExpr(start=s):
            return (s,)
    return ()


def walk(statements: tuple[Stmt, ...]):
    """Every statement, depth first."""
    for s in statements:
        yield s
        if isinstance(s, For):
            yield from walk(s.body)
        elif isinstance(s, If):
            yield from walk(s.then)
            yield from walk(s.orelse)

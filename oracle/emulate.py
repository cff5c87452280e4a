"""The oracle emulator: runs the tile IR block by block with numpy, lane validity included.

TEST INFRASTRUCTURE ONLY (see oracle/numerics.py).

Restates krn's Python emulator for the tile path (reference src/krn/emulator/emulate.py): tile loads read zero outside
the tensor and mark those lanes invalid (load_tile/tile_valid 248-261), elementwise results are valid where every
operand is, reductions skip invalid lanes and start from the identity (reduce_valid 284-292), a product counts invalid
lanes as zero and leaves a row or column with no valid lane invalid (accumulate 305-324), and stores skip invalid
lanes and elements outside the tensor (store_tile 263-275). Accumulation is one fused multiply-add per k in k order
(fused 347-385). bf16 tiles live as float32 values rounded to bf16 (np_dtype 140-141).

Beyond the reference emulator, which refuses fp8 products (emulate.py:980-981) and has no int8 product: fp8 operands
are decoded exactly to float32 first, and int8 operands accumulate exactly in int32.
"""

from collections.abc import Sequence

import math

import numpy as np

from krn_amd.compiler import ir
from krn_amd.compiler.space import geometry, runtime_args
from krn_amd.dtypes import BF16, BOOL, F16, I32, NUMPY, PY_FLOAT, PY_INT, Dtype
from krn_amd.frontend import Blocks
from oracle.numerics import bf16_round, e4m3_decode, e4m3_encode, fma32


def tile_dtype(dtype: Dtype) -> np.dtype:
    """How the emulator holds a tile element: bf16 as float32, fp8 as its uint8 code."""
    if dtype == BF16:
        return np.dtype(np.float32)
    return NUMPY[dtype]


def host_values(array: np.ndarray, dtype: Dtype) -> np.ndarray:
    """A tensor's storage as tile elements (bf16 words become float32 values)."""
    if dtype == BF16 and array.dtype == np.uint16:
        return (array.astype(np.uint32) << 16).view(np.float32)
    return array


def to_storage(values: np.ndarray, dtype: Dtype) -> np.ndarray:
    if dtype == BF16:
        return (bf16_round(values).view(np.uint32) >> 16).astype(np.uint16)
    return values.astype(NUMPY[dtype])


def convert(values: np.ndarray, src: Dtype, dst: Dtype) -> np.ndarray:
    """`.to(dst)`: an fp8 code decodes to float32 first; an fp8 result is encoded last."""
    if src == dst:
        return values
    if src.is_narrow:
        values = e4m3_decode(values)
    if dst.is_narrow:
        return e4m3_encode(np.asarray(values, np.float32))
    if dst == BF16:
        return bf16_round(np.asarray(values, np.float32))
    if dst == BOOL:
        return np.asarray(values) != 0
    with np.errstate(all="ignore"):
        return np.asarray(values).astype(tile_dtype(dst))


def scalar_convert(value: object, dtype: Dtype) -> object:
    if dtype == PY_INT:
        return int(value)
    if dtype == PY_FLOAT:
        return float(value)
    if dtype == BOOL:
        return bool(value)
    if dtype.is_float:
        return convert(np.asarray(value, np.float64), PY_FLOAT, dtype)[()]
    bits = dtype.bits
    v = int(value) & ((1 << bits) - 1)
    return v - (1 << bits) if dtype.kind.value == "sint" and v >> (bits - 1) else v


def regions(shape, starts, extents):
    lows = [max(s, 0) for s in starts]
    highs = [max(min(s + e, n), lo) for s, e, n, lo in zip(starts, extents, shape, lows)]
    inside = tuple(slice(lo, hi) for lo, hi in zip(lows, highs))
    local = tuple(slice(lo - s, hi - s) for s, lo, hi in zip(starts, lows, highs))
    return inside, local


class Block:
    """The state of one block: tile variables with their validity, scalar locals."""

    def __init__(self, kernel: ir.Kernel, tensors: dict, scalars: dict, index: tuple[int, int, int]):
        self.kernel, self.tensors, self.scalars = kernel, tensors, scalars
        self.index = dict(zip("xyz", index))
        self.tiles: dict[str, np.ndarray] = {}
        self.valid: dict[str, np.ndarray] = {}
        self.locals: dict[str, object] = {}

    # statements

    def run(self, statements: Sequence[ir.Stmt]) -> None:
        for s in statements:
            getattr(self, f"stmt_{type(s).__name__}")(s)

    def stmt_TileAssign(self, s: ir.TileAssign) -> None:
        value, valid = self.tile(s.value)
        self.tiles[s.var.name] = np.array(np.broadcast_to(value, s.var.shape), tile_dtype(s.var.dtype))
        self.valid[s.var.name] = np.array(np.broadcast_to(valid, s.var.shape))

    def stmt_TileStore(self, s: ir.TileStore) -> None:
        value, valid = self.tile(s.value)
        array = self.tensors[s.tensor.name]
        starts = [int(self.scalar(sl.start)) for sl in s.slices]
        extents = [sl.extent for sl in s.slices]
        values = np.broadcast_to(value, s.value.shape).reshape(extents)
        keep = np.broadcast_to(valid, s.value.shape).reshape(extents)
        inside, local = regions(array.shape, starts, extents)
        target = array[inside]
        stored = to_storage(values[local], s.tensor.type.dtype)
        target[keep[local]] = stored[keep[local]]
        array[inside] = target

    def stmt_Accumulate(self, s: ir.Accumulate) -> None:
        lhs, lv = self.tile(s.lhs)
        rhs, rv = self.tile(s.rhs)
        lhs = np.where(np.broadcast_to(lv, s.lhs.shape), lhs, 0)
        rhs = np.where(np.broadcast_to(rv, s.rhs.shape), rhs, 0)
        acc = self.tiles[s.acc.name]
        if s.acc.dtype == I32:
            total = acc.astype(np.int64) + lhs.astype(np.int64) @ rhs.astype(np.int64)
            acc[...] = ((total + 2**31) % 2**32 - 2**31).astype(np.int32)
        else:
            if s.lhs.dtype.is_narrow:
                lhs, rhs = e4m3_decode(lhs), e4m3_decode(rhs)
            left, right = lhs.astype(np.float32), rhs.astype(np.float32)
            if np.isfinite(left).all() and np.isfinite(right).all():
                for k in range(left.shape[1]):
                    acc[...] = fma32(left[:, k, None], right[None, k, :], acc)
            else:  # non-finite operands: a float64 product is exact enough to carry inf/nan as the hardware does
                for k in range(left.shape[1]):
                    acc[...] = (left[:, k, None].astype(np.float64) * right[None, k, :] + acc).astype(np.float32)
        valid = self.valid[s.acc.name]
        valid &= np.broadcast_to(lv, s.lhs.shape).any(axis=1, keepdims=True)
        valid &= np.broadcast_to(rv, s.rhs.shape).any(axis=0, keepdims=True)

    def stmt_For(self, s: ir.For) -> None:
        lo, hi = int(self.scalar(s.lo)), int(self.scalar(s.hi))
        for i in range(lo, hi, s.step):
            self.locals[s.var.name] = i
            self.run(s.body)

    def stmt_If(self, s: ir.If) -> None:
        self.run(s.then if self.scalar(s.cond) else s.orelse)

    def stmt_Assign(self, s: ir.Assign) -> None:
        self.locals[s.var.name] = self.scalar(s.value)

    # scalar expressions

    def scalar(self, e: ir.Expr) -> object:
        match e:
            case ir.Const(value=v):
                return scalar_convert(v, e.dtype)
            case ir.Var(name=n):
                return self.locals[n]
            case ir.Param(name=n):
                return self.scalars[n]
            case ir.Dim(tensor=t, axis=a):
                return self.tensors[t.name].shape[a]
            case ir.BlockIndex(axis=a):
                return self.index[a]
            case ir.Cast(operand=o):
                return scalar_convert(self.scalar(o), e.dtype)
            case ir.Unary(op=ir.Op.NEG, operand=o):
                return -self.scalar(o)
            case ir.Binary(op=op, lhs=a, rhs=b):
                x, y = self.scalar(a), self.scalar(b)
                if op is ir.Op.DIV and e.dtype.is_int or (op is ir.Op.DIV and e.dtype == PY_INT):
                    return int(x / y) if y else 0
                result = SCALAR_OPS[op](x, y)
                return result if op in ir.COMPARISONS else scalar_convert(result, e.dtype)
        raise NotImplementedError(f"scalar {type(e).__name__}")

    # tile expressions: (values, validity)

    def tile(self, e: ir.Expr) -> tuple[np.ndarray, np.ndarray]:
        if not e.shape:
            value = self.scalar(e)
            if e.dtype.is_float and e.dtype != PY_FLOAT:
                value = np.asarray(value, tile_dtype(e.dtype))
            return np.asarray(value), np.bool_(True)
        return getattr(self, f"tile_{type(e).__name__}")(e)

    def tile_Var(self, e: ir.Var):
        return self.tiles[e.name], self.valid[e.name]

    def tile_Zeros(self, e: ir.Zeros):
        return np.zeros(e.shape, tile_dtype(e.dtype)), np.bool_(True)

    def tile_TileLoad(self, e: ir.TileLoad):
        array = host_values(self.tensors[e.tensor.name], e.tensor.type.dtype)
        starts = [int(self.scalar(sl.start)) for sl in e.slices]
        extents = [sl.extent for sl in e.slices]
        tile = np.zeros(extents, tile_dtype(e.dtype))
        valid = np.zeros(extents, bool)
        inside, local = regions(array.shape, starts, extents)
        tile[local] = array[inside]
        valid[local] = True
        return tile.reshape(e.shape), valid.reshape(e.shape)

    def tile_Transpose(self, e: ir.Transpose):
        value, valid = self.tile(e.operand)
        return np.swapaxes(value, 0, 1), np.swapaxes(np.broadcast_to(valid, e.operand.shape), 0, 1)

    def tile_Arange(self, e: ir.Arange):
        start = int(self.scalar(e.start))
        ramp = np.arange(start, start + e.shape[e.axis], dtype=np.int32)
        shape = [-1 if a == e.axis else 1 for a in range(len(e.shape))]
        return np.broadcast_to(ramp.reshape(shape), e.shape).copy(), np.bool_(True)

    def tile_Cast(self, e: ir.Cast):
        value, valid = self.tile(e.operand)
        return convert(value, e.operand.dtype, e.dtype), valid

    def tile_Unary(self, e: ir.Unary):
        value, valid = self.tile(e.operand)
        return self.round(-value, e.dtype), valid

    def tile_Binary(self, e: ir.Binary):
        (a, av), (b, bv) = self.tile(e.lhs), self.tile(e.rhs)
        with np.errstate(all="ignore"):
            if e.op is ir.Op.DIV and e.lhs.dtype.is_int:
                out = np.where(b != 0, np.trunc(a / np.where(b != 0, b, 1)), 0).astype(a.dtype)
            else:
                out = TILE_OPS[e.op](a, b)
        if e.op not in ir.COMPARISONS:
            out = self.round(out, e.dtype)
        return out, av & bv

    def tile_Math(self, e: ir.Math):
        parts = [self.tile(a) for a in e.args]
        with np.errstate(all="ignore"):
            out = MATH[e.fn](*(p[0] for p in parts))
        valid = np.bool_(True)
        for _, v in parts:
            valid = valid & v
        return self.round(out, e.dtype), valid

    def tile_Select(self, e: ir.Select):
        (c, cv), (t, tv), (f, fv) = self.tile(e.cond), self.tile(e.then), self.tile(e.orelse)
        return self.round(np.where(c, t, f), e.dtype), cv & tv & fv

    def tile_Reduce(self, e: ir.Reduce):
        value, valid = self.tile(e.operand)
        where = np.broadcast_to(valid, e.operand.shape)
        initial = {
            ir.Reduction.MAX: -np.inf if value.dtype.kind == "f" else np.iinfo(value.dtype).min,
            ir.Reduction.MIN: np.inf if value.dtype.kind == "f" else np.iinfo(value.dtype).max,
            ir.Reduction.SUM: 0,
        }[e.op]
        function = {ir.Reduction.MAX: np.max, ir.Reduction.MIN: np.min, ir.Reduction.SUM: np.sum}[e.op]
        out = function(value, axis=e.axis, keepdims=e.keepdims, where=where, initial=initial)
        any_valid = where.any(axis=e.axis, keepdims=e.keepdims)
        return self.round(out.astype(tile_dtype(e.dtype)), e.dtype), any_valid

    def round(self, value: np.ndarray, dtype: Dtype) -> np.ndarray:
        if dtype == BF16:
            return bf16_round(np.asarray(value, np.float32))
        if dtype == BOOL:
            return np.asarray(value, bool)
        return np.asarray(value).astype(tile_dtype(dtype), copy=False)


SCALAR_OPS = {
    ir.Op.ADD: lambda a, b: a + b, ir.Op.SUB: lambda a, b: a - b, ir.Op.MUL: lambda a, b: a * b,
    ir.Op.DIV: lambda a, b: a / b, ir.Op.MOD: lambda a, b: a % b, ir.Op.LT: lambda a, b: a < b,
    ir.Op.LE: lambda a, b: a <= b, ir.Op.GT: lambda a, b: a > b, ir.Op.GE: lambda a, b: a >= b,
    ir.Op.EQ: lambda a, b: a == b, ir.Op.NE: lambda a, b: a != b, ir.Op.AND: lambda a, b: a and b,
    ir.Op.OR: lambda a, b: a or b,
}  # fmt: skip
TILE_OPS = {
    ir.Op.ADD: np.add, ir.Op.SUB: np.subtract, ir.Op.MUL: np.multiply, ir.Op.DIV: np.divide, ir.Op.MOD: np.fmod,
    ir.Op.LT: np.less, ir.Op.LE: np.less_equal, ir.Op.GT: np.greater, ir.Op.GE: np.greater_equal,
    ir.Op.EQ: np.equal, ir.Op.NE: np.not_equal, ir.Op.AND: np.logical_and, ir.Op.OR: np.logical_or,
}  # fmt: skip
_erf = np.vectorize(math.erf, otypes=[np.float64])
MATH = {
    ir.Fn.EXP: np.exp, ir.Fn.EXP2: np.exp2, ir.Fn.LOG: np.log, ir.Fn.LOG2: np.log2, ir.Fn.SQRT: np.sqrt,
    ir.Fn.RSQRT: lambda x: 1 / np.sqrt(x), ir.Fn.ABS: np.abs, ir.Fn.TANH: np.tanh,
    ir.Fn.RELU: lambda x: np.maximum(x, 0), ir.Fn.MAXIMUM: np.maximum, ir.Fn.MINIMUM: np.minimum,
    # reference emulator/emulate.py:373-384: erf in float64 rounded to the operand's type, the rest in that type
    ir.Fn.ERF: lambda x: _erf(x).astype(x.dtype),
    ir.Fn.GELU: lambda x: x.dtype.type(0.5) * x * (x.dtype.type(1) + _erf(x * x.dtype.type(0.7071067811865476)).astype(x.dtype)),
    ir.Fn.SILU: lambda x: x / (x.dtype.type(1) + np.exp(-x)),
    ir.Fn.SIGMOID: lambda x: x.dtype.type(1) / (x.dtype.type(1) + np.exp(-x)),
}  # fmt: skip


def run(kernel: ir.Kernel, launch: Blocks | None, args: Sequence[object]) -> None:
    """Run `kernel` over every block of `launch` (inferred from the body when None). Tensor arguments are numpy
    arrays in storage form (bf16 as uint16 words, fp8 as uint8 codes) and are written in place."""
    values = runtime_args(kernel, args)
    tensors, scalars = {}, {}
    for (name, kind), value in zip(kernel.params, values):
        if isinstance(kind, ir.TensorType):
            if not isinstance(value, np.ndarray) or value.ndim != kind.rank:
                raise TypeError(f"{kernel.name}: `{name}` needs a rank-{kind.rank} array")
            tensors[name] = value
        else:
            scalars[name] = scalar_convert(value, kind)
    grid = launch if launch is not None else geometry(kernel, values)
    for z in range(grid.z):
        for y in range(grid.y):
            for x in range(grid.x):
                Block(kernel, tensors, scalars, (x, y, z)).run(kernel.body)

"""Capture a `@kernel` function from its source file into the tile IR, without executing it.

This re-creates the subset of krn's capture that the tile path uses (reference src/krn/compiler/capture.py:427 and
the rules cited per method): tensor slices as tiles, `block.tile`/`block.index`, `zeros`, `arange`, `where`,
comparisons, fluent elementwise methods, `keepdims` reductions, `.to(dtype)`, `.transpose()`, `acc += a @ b` and the
bare product `a @ b`, `for ... in range(...)` and `pipelined(...)` loops, and `if` on compile-time constants or
runtime scalars. `Const` fields of a `@struct` configuration are folded. Anything else is refused with a
`CaptureError` that names the user's file and line.

Beyond the reference: an int8 x int8 product accumulates into an int32 tile (the reference refuses int8 `@`,
capture.py:3193-3201), and fp8/int8 operands may be a direct tile load or the transpose of one (the reference
accepts only direct loads, capture.py:3185-3191), which is how a `B^T` weight layout is written.
"""

import ast
import math
from dataclasses import dataclass
from pathlib import Path

from krn_amd import dtypes as D
from krn_amd.dtypes import BOOL, F32, I8, I32, PY_FLOAT, PY_INT, Dtype
from krn_amd.compiler.ir import (
    COMPARISONS,
    Accumulate,
    Arange,
    Assign,
    Binary,
    BlockIndex,
    Cast,
    Const,
    Dim,
    Expr,
    Fn,
    For,
    If,
    Kernel,
    Math,
    Op,
    Param,
    Reduce,
    Reduction,
    Select,
    SliceExpr,
    SliceType,
    Stmt,
    TensorRef,
    TensorType,
    TileAssign,
    TileLoad,
    TileStore,
    TileType,
    Transpose,
    Unary,
    Var,
    Zeros,
    tile_shape,
)


class CaptureError(ValueError):
    """A kernel body outside the captured subset, or a type error in it, at a line of the user's file."""


class TargetError(CaptureError):
    """An unavailable target feature, with the alternative to use (reference compiler/errors.py:56-62)."""

    def __init__(self, feature: str, target: str, reason: str, instead: str) -> None:
        self.feature, self.target, self.reason, self.instead = feature, target, reason, instead
        super().__init__(f"{feature} is not available on {target}: {reason.rstrip('.')}. "
                         f"Instead: {instead.rstrip('.')}.")


TENSOR_RANKS = {"Matrix": 2, "Vector": 1, "Tensor3": 3}
ARITHMETIC = {"add": Op.ADD, "sub": Op.SUB, "mul": Op.MUL, "div": Op.DIV, "truediv": Op.DIV}
UNARY_MATH = {
    "exp": Fn.EXP, "exp2": Fn.EXP2, "log": Fn.LOG, "log2": Fn.LOG2, "sqrt": Fn.SQRT, "rsqrt": Fn.RSQRT,
    "abs": Fn.ABS, "tanh": Fn.TANH, "relu": Fn.RELU, "gelu": Fn.GELU, "silu": Fn.SILU, "sigmoid": Fn.SIGMOID,
    "erf": Fn.ERF,
}  # fmt: skip
BINARY_MATH = {"maximum": Fn.MAXIMUM, "minimum": Fn.MINIMUM}
NORMALIZING = ("softmax", "log_softmax")  # take `axis` and keep the shape
BINOPS = {ast.Add: Op.ADD, ast.Sub: Op.SUB, ast.Mult: Op.MUL, ast.Div: Op.DIV, ast.Mod: Op.MOD}
CMPOPS = {ast.Lt: Op.LT, ast.LtE: Op.LE, ast.Gt: Op.GT, ast.GtE: Op.GE, ast.Eq: Op.EQ, ast.NotEq: Op.NE}


@dataclass(frozen=True)
class Packed:
    """A tuple of values, as `block.tile(bm, bn)` returns."""

    items: tuple


@dataclass(frozen=True)
class Config:
    """A configuration parameter whose fields are all compile-time constants."""

    name: str
    values: dict


class _BlockIndexValue:
    """The value of `block.index()`; its `.x/.y/.z` are the grid coordinates."""


def dotted(node: ast.AST) -> str:
    if isinstance(node, ast.Name):
        return node.id
    if isinstance(node, ast.Attribute):
        return f"{dotted(node.value)}.{node.attr}"
    return ""


def dtype_name(node: ast.AST) -> str | None:
    """The element type an annotation or dtype argument names: `T.f16`, `f16`, `krn.T.bf16`, `int`, `float`."""
    name = dotted(node).rsplit(".", 1)[-1]
    if name in D.BY_NAME:
        return name
    if name in ("int", "float", "bool"):
        return name
    return None


def struct_defaults(module: ast.Module) -> dict[str, dict[str, object]]:
    """Default values of the `Const` fields of each `@struct` class in the file."""
    found: dict[str, dict[str, object]] = {}
    for node in module.body:
        if isinstance(node, ast.ClassDef) and any(dotted(d).endswith("struct") for d in node.decorator_list):
            fields: dict[str, object] = {}
            for item in node.body:
                if isinstance(item, ast.AnnAssign) and isinstance(item.target, ast.Name):
                    if item.value is not None:
                        fields[item.target.id] = ast.literal_eval(item.value)
                    else:
                        fields[item.target.id] = None
            found[node.name] = fields
    return found


class Capture:
    def __init__(self, path: Path, source: str, fn: ast.FunctionDef, consts: dict, dtypes: dict, structs: dict):
        self.path, self.source, self.fn = path, source, fn
        self.consts, self.dtype_overrides, self.structs = consts, dtypes, structs
        self.env: dict[str, object] = {}
        self.params: list[tuple[str, Dtype | TensorType]] = []
        self.tiles: list[Var] = []
        self.out: list[Stmt] = []
        self.space: dict[str, tuple[int, list[Expr]]] = {}
        self.counter = 0

    # ---- errors and helpers

    def error(self, node: ast.AST, message: str) -> CaptureError:
        line = getattr(node, "lineno", self.fn.lineno)
        text = self.source.splitlines()[line - 1].strip() if 0 < line <= len(self.source.splitlines()) else ""
        return CaptureError(f"{self.path}:{line}: {message}\n    {text}")

    def fresh(self, stem: str) -> str:
        self.counter += 1
        return f"_{stem}{self.counter}"

    # ---- parameters

    def parameters(self) -> None:
        for arg in self.fn.args.args:
            name, annotation = arg.arg, arg.annotation
            if annotation is None:
                raise self.error(arg, f"parameter `{name}` needs a type annotation")
            if name in self.consts:
                self.env[name] = Config(name, dict(self.consts[name]))
                continue
            base = annotation.value if isinstance(annotation, ast.Subscript) else annotation
            base_name = dotted(base).rsplit(".", 1)[-1]
            if base_name in self.structs:
                self.env[name] = Config(name, dict(self.structs[base_name]))
                continue
            if isinstance(annotation, ast.Subscript) and base_name in ("Tensor", "Matrix", "Vector", "Tensor3"):
                items = annotation.slice.elts if isinstance(annotation.slice, ast.Tuple) else [annotation.slice]
                element = dtype_name(items[0])
                generic = element is None and isinstance(items[0], ast.Name)  # `Matrix[F]`, F a type variable
                if generic and name not in self.dtype_overrides:
                    raise self.error(arg, f"tensor `{name}` is generic over {items[0].id}: its element type comes from "
                                          "the argument, and none was given")
                if not generic and (element is None or element in ("int", "float", "bool")):
                    raise self.error(arg, f"tensor `{name}` needs an element type such as T.f32")
                rank = TENSOR_RANKS.get(base_name, len(items) - 1)
                if rank < 1:
                    raise self.error(arg, f"tensor `{name}` needs at least one axis: Tensor[T.f32, int, int]")
                dtype = self.dtype_overrides[name] if generic else self.dtype_overrides.get(name, D.BY_NAME[element])
                kind = TensorType(dtype, rank)
                self.params.append((name, kind))
                self.env[name] = TensorRef(name, kind)
                continue
            element = dtype_name(annotation)
            if element is None:
                raise self.error(arg, f"parameter `{name}` has an annotation the tile path does not capture")
            dtype = {"int": D.I64, "float": F32, "bool": BOOL}.get(element) or D.BY_NAME[element]
            dtype = self.dtype_overrides.get(name, dtype)
            self.params.append((name, dtype))
            self.env[name] = Param(dtype, name, line=arg.lineno)

    # ---- statements

    def block(self, statements: list[ast.stmt]) -> tuple[Stmt, ...]:
        saved, self.out = self.out, []
        for statement in statements:
            self.statement(statement)
        body, self.out = tuple(self.out), saved
        return body

    def statement(self, node: ast.stmt) -> None:
        match node:
            case ast.Expr(value=ast.Constant(value=str())):
                return  # a docstring
            case ast.Pass():
                return
            case ast.Assign(targets=[target], value=value):
                self.assign(target, value, node)
            case ast.AnnAssign(target=target, value=value) if value is not None:
                self.assign(target, value, node)
            case ast.AugAssign():
                self.augmented(node)
            case ast.For():
                self.loop(node)
            case ast.If():
                self.conditional(node)
            case _:
                raise self.error(node, f"`{type(node).__name__}` statements are not captured on the tile path")

    def assign(self, target: ast.expr, value: ast.expr, node: ast.stmt) -> None:
        if isinstance(target, ast.Tuple):
            if isinstance(value, ast.Tuple):
                values = [self.expr_or_value(v) for v in value.elts]
            else:
                packed = self.expr_or_value(value)
                if not isinstance(packed, Packed):
                    raise self.error(node, "only a tuple or `block.tile(bm, bn)` unpacks into several names")
                values = list(packed.items)
            if len(values) != len(target.elts):
                raise self.error(node, f"{len(target.elts)} names for {len(values)} values")
            for name, v in zip(target.elts, values):
                self.bind(name, v, node)
            return
        if isinstance(target, ast.Subscript):
            self.store(target, self.expr(value), node)
            return
        self.bind(target, self.expr_or_value(value), node)

    def bind(self, target: ast.expr, value: object, node: ast.AST) -> None:
        if not isinstance(target, ast.Name):
            raise self.error(node, "assignments bind plain names")
        name = target.id
        if isinstance(value, Expr) and isinstance(value.type, TileType):
            current = self.env.get(name)
            if isinstance(current, Var) and current.type == value.type:
                self.out.append(TileAssign(current, value, line=node.lineno))
                return
            var = Var(value.type, self.fresh(name) if isinstance(current, Var) else name, line=node.lineno)
            self.tiles.append(var)
            self.out.append(TileAssign(var, value, line=node.lineno))
            self.env[name] = var
            return
        self.env[name] = value  # scalars, slices, packed tuples: immutable bindings

    def augmented(self, node: ast.AugAssign) -> None:
        if not isinstance(node.target, ast.Name):
            raise self.error(node, "augmented assignment updates a tile variable")
        acc = self.env.get(node.target.id)
        if isinstance(node.op, ast.Add) and isinstance(node.value, ast.BinOp) and isinstance(node.value.op, ast.MatMult):
            if not (isinstance(acc, Var) and isinstance(acc.type, TileType)):
                raise self.error(node, "the target of `+= a @ b` must be a tile variable")
            self.accumulate(node, acc, self.expr(node.value.left), self.expr(node.value.right))
            return
        op = BINOPS.get(type(node.op))
        if op is None or not isinstance(acc, Var) or not isinstance(acc.type, TileType):
            raise self.error(node, "augmented assignment is captured for tile variables and + - * /")
        new = self.binary(op, acc, self.expr(node.value), node)
        if new.type != acc.type:
            raise self.error(node, f"`{node.target.id}` is {acc.type.dtype}{list(acc.shape)}, the update is "
                             f"{new.dtype}{list(new.shape)}")
        self.out.append(TileAssign(acc, new, line=node.lineno))

    def accumulate(self, node: ast.AST, acc: Var, lhs: Expr, rhs: Expr) -> None:
        """`acc += lhs @ rhs` (reference capture.py:3170-3211): float operands f16/bf16/f32 (a mix is widened to
        f32), fp8 pairs kept as raw loads, and int8 pairs into an int32 accumulator."""
        if not (len(lhs.shape) == 2 and len(rhs.shape) == 2):
            raise self.error(node, f"`@` needs two rank-2 tiles, got {lhs.type} and {rhs.type}")
        (m, k), (k2, n) = lhs.shape, rhs.shape
        if k != k2:
            raise self.error(node, f"inner dimensions of `@` differ: {lhs.shape} @ {rhs.shape}")
        operands = (lhs.dtype, rhs.dtype)
        raw = all(d.is_narrow for d in operands) or all(d == I8 for d in operands)
        if raw:
            for operand in (lhs, rhs):
                inner = operand.operand if isinstance(operand, Transpose) else operand
                if not isinstance(inner, TileLoad):
                    raise self.error(node, f"{operand.dtype} matrix operands must be direct tile loads (or their "
                                     "transpose); no expression decode exists")
            want = I32 if operands[0] == I8 else F32
        else:
            if any(not d.is_float or d.bits not in (16, 32) for d in operands):
                raise self.error(node, f"`@` f32 accumulator needs lossless operands (f16, bf16 or f32), got "
                                 f"{operands[0]} and {operands[1]}")
            want = F32
            if operands[0] != operands[1]:
                lhs, rhs = self.cast(lhs, F32), self.cast(rhs, F32)
        if acc.type != TileType(want, (m, n)):
            raise self.error(node, f"the accumulator is {acc.dtype} {acc.shape}, the product is {want} {(m, n)}")
        self.out.append(Accumulate(acc, lhs, rhs, line=getattr(node, "lineno", 0)))

    def product(self, node: ast.BinOp) -> Var:
        """A bare `a @ b`: the product into a fresh zeroed accumulator (reference capture.py:3157-3168)."""
        lhs, rhs = self.expr(node.left), self.expr(node.right)
        if not (len(lhs.shape) == 2 and len(rhs.shape) == 2):
            raise self.error(node, f"`@` needs two rank-2 tiles, got {lhs.type} and {rhs.type}")
        want = I32 if lhs.dtype == I8 and rhs.dtype == I8 else F32
        shape = (lhs.shape[0], rhs.shape[1])
        acc = Var(TileType(want, shape), self.fresh("product"), line=node.lineno)
        self.tiles.append(acc)
        self.out.append(TileAssign(acc, Zeros(TileType(want, shape)), line=node.lineno))
        self.accumulate(node, acc, lhs, rhs)
        return acc

    def store(self, target: ast.Subscript, value: Expr, node: ast.stmt) -> None:
        tensor = self.expr_or_value(target.value)
        if not isinstance(tensor, TensorRef):
            raise self.error(node, "subscript assignment writes a tensor parameter")
        slices = self.slices(tensor, target.slice, node)
        if all(s.squeeze for s in slices):
            raise self.error(node, "scalar element stores are the SIMT path, not captured on the tile path")
        shape = tile_shape(slices)
        if value.shape != shape:
            raise self.error(node, f"storing a {list(value.shape)} tile into a {list(shape)} slice")
        if value.dtype != tensor.type.dtype:
            raise self.error(node, f"storing {value.dtype} into a {tensor.type.dtype} tensor; convert with .to(...)")
        for axis, s in enumerate(slices):
            if (tiled := self.block_tile_axis(s)) is not None:
                grid, size = tiled
                self.space.setdefault(grid, (size, []))[1].append(Dim(PY_INT, tensor, axis))
        self.out.append(TileStore(tensor, slices, value, line=node.lineno))

    def block_tile_axis(self, s: SliceExpr) -> tuple[str, int] | None:
        match s.start:
            case Binary(op=Op.MUL, lhs=BlockIndex(axis=axis), rhs=Const(value=size)) if not s.squeeze:
                return axis, int(size)
        return None

    def loop(self, node: ast.For) -> None:
        if node.orelse or not isinstance(node.target, ast.Name) or not isinstance(node.iter, ast.Call):
            raise self.error(node, "loops are `for name in range(...)` or `for ks in pipelined(extent, tile)`")
        call, name = node.iter, node.target.id
        function = dotted(call.func).rsplit(".", 1)[-1]
        if function == "range":
            args = [self.expr(a) for a in call.args]
            if not 1 <= len(args) <= 3 or call.keywords:
                raise self.error(node, "`range` takes one to three positional arguments")
            lo, hi = (Const(PY_INT, 0), args[0]) if len(args) == 1 else (args[0], args[1])
            step = 1
            if len(args) == 3:
                if not isinstance(args[2], Const) or int(args[2].value) <= 0:
                    raise self.error(node, "a loop step must be a positive compile-time constant")
                step = int(args[2].value)
            var = Var(PY_INT, self.fresh(name), line=node.lineno)
            previous = self.env.get(name)
            self.env[name] = var
            body = self.block(node.body)
            self.restore(name, previous)
            self.out.append(For(var, self.scalar(lo, node), self.scalar(hi, node), step, body, line=node.lineno))
            return
        if function == "pipelined":
            if not call.args:
                raise self.error(call, "`pipelined(extent, tile)` is missing the extent")
            extent = self.expr(call.args[0])
            args = list(call.args[1:])
            keywords = {k.arg: k.value for k in call.keywords}
            tile_node = args[0] if args else keywords.get("tile")
            if tile_node is None:
                raise self.error(call, "`pipelined(extent, tile)` is missing the tile size")
            size = self.constant(tile_node, "a tile size")
            stages = int(self.constant(keywords["stages"], "a stage count")) if (
                "stages" in keywords and not dotted(keywords["stages"]).endswith("AUTO")
            ) else 0
            if int(size) <= 0:
                raise self.error(call, "`pipelined` needs a positive tile")
            start = Var(PY_INT, self.fresh(f"{name}_start"), line=node.lineno)
            previous = self.env.get(name)
            self.env[name] = SliceExpr(SliceType(int(size)), start, line=node.lineno)
            body = self.block(node.body)
            self.restore(name, previous)
            self.out.append(For(start, Const(PY_INT, 0), self.scalar(extent, node), int(size), body,
                                pipelined=True, stages=stages, line=node.lineno))
            return
        raise self.error(node, f"`for` over `{function}` is not captured; use range(...) or pipelined(...)")

    def restore(self, name: str, previous: object) -> None:
        if previous is None:
            self.env.pop(name, None)
        else:
            self.env[name] = previous

    def conditional(self, node: ast.If) -> None:
        cond = self.expr(node.test)
        if isinstance(cond, Const):
            for statement in node.body if cond.value else node.orelse:
                self.statement(statement)
            return
        if cond.shape:
            raise self.error(node, "an `if` condition is a scalar; use `where` for tiles")
        self.out.append(If(cond, self.block(node.body), self.block(node.orelse), line=node.lineno))

    # ---- expressions

    def expr(self, node: ast.expr) -> Expr:
        value = self.expr_or_value(node)
        if not isinstance(value, Expr):
            raise self.error(node, f"`{ast.unparse(node)}` is not a value")
        return value

    def expr_or_value(self, node: ast.expr) -> object:
        match node:
            case ast.Constant(value=bool() as v):
                return Const(BOOL, v, line=node.lineno)
            case ast.Constant(value=int() as v):
                return Const(PY_INT, v, line=node.lineno)
            case ast.Constant(value=float() as v):
                return Const(PY_FLOAT, v, line=node.lineno)
            case ast.Name(id=name):
                if name in self.env:
                    return self.env[name]
                if name in ("math",):
                    return name
                raise self.error(node, f"`{name}` is not defined in the kernel")
            case ast.Attribute():
                return self.attribute(node)
            case ast.Subscript():
                return self.subscript(node)
            case ast.BinOp(op=ast.MatMult()):
                return self.product(node)
            case ast.BinOp(op=op, left=left, right=right) if type(op) in BINOPS:
                return self.binary(BINOPS[type(op)], self.expr(left), self.expr(right), node)
            case ast.UnaryOp(op=ast.USub(), operand=operand):
                value = self.expr(operand)
                if isinstance(value, Const):
                    return Const(value.dtype, -value.value, line=node.lineno)
                return Unary(value.type, Op.NEG, value, line=node.lineno)
            case ast.UnaryOp(op=ast.Not(), operand=operand):
                value = self.expr(operand)
                if isinstance(value, Const):
                    return Const(BOOL, not value.value, line=node.lineno)
                raise self.error(node, "`not` is captured on constants only")
            case ast.Compare(left=left, ops=[op], comparators=[right]) if type(op) in CMPOPS:
                return self.binary(CMPOPS[type(op)], self.expr(left), self.expr(right), node)
            case ast.BoolOp():
                values = [self.expr(v) for v in node.values]
                if all(isinstance(v, Const) for v in values):
                    result = all(v.value for v in values) if isinstance(node.op, ast.And) else any(
                        v.value for v in values)
                    return Const(BOOL, result, line=node.lineno)
                raise self.error(node, "`and`/`or` are captured on constants only; use `&` on tiles")
            case ast.Call():
                return self.call(node)
            case ast.Tuple(elts=elts):
                return Packed(tuple(self.expr_or_value(e) for e in elts))
        raise self.error(node, f"`{ast.unparse(node)}` is not captured on the tile path")

    def attribute(self, node: ast.Attribute) -> object:
        base = self.expr_or_value(node.value) if not isinstance(node.value, ast.Name) or node.value.id in self.env \
            else node.value.id
        if isinstance(base, Config):
            if node.attr not in base.values:
                raise self.error(node, f"configuration `{base.name}` has no field `{node.attr}`")
            value = base.values[node.attr]
            if isinstance(value, bool):
                return Const(BOOL, value, line=node.lineno)
            if isinstance(value, int):
                return Const(PY_INT, value, line=node.lineno)
            if isinstance(value, float):
                return Const(PY_FLOAT, value, line=node.lineno)
            raise self.error(node, f"field `{node.attr}` = {value!r} is not a number")
        if isinstance(base, _BlockIndexValue):
            if node.attr not in "xyz" or len(node.attr) != 1:
                raise self.error(node, "`block.index()` has .x, .y and .z")
            return BlockIndex(PY_INT, node.attr, line=node.lineno)
        if node.attr == "shape" and isinstance(base, (TensorRef, Expr)):
            return ("shape", base)
        if base == "math" and node.attr in ("pi", "e"):
            return Const(PY_FLOAT, getattr(math, node.attr), line=node.lineno)
        raise self.error(node, f"`{ast.unparse(node)}` is not captured on the tile path")

    def subscript(self, node: ast.Subscript) -> object:
        base = self.expr_or_value(node.value)
        if isinstance(base, tuple) and base and base[0] == "shape":
            axis = self.constant(node.slice, "an axis")
            owner = base[1]
            if isinstance(owner, TensorRef):
                if not -owner.type.rank <= int(axis) < owner.type.rank:
                    raise self.error(node, f"tensor `{owner.name}` has {owner.type.rank} axes, no axis {axis}")
                return Dim(PY_INT, owner, int(axis) % owner.type.rank, line=node.lineno)
            rank = len(owner.shape)
            if not -rank <= int(axis) < rank:
                raise self.error(node, f"the tile has {rank} axes, no axis {axis}")
            return Const(PY_INT, owner.shape[int(axis)], line=node.lineno)
        if isinstance(base, TensorRef):
            slices = self.slices(base, node.slice, node)
            if all(s.squeeze for s in slices):
                raise self.error(node, "scalar element loads are the SIMT path, not captured on the tile path")
            return TileLoad(TileType(base.type.dtype, tile_shape(slices)), base, slices, line=node.lineno)
        raise self.error(node, f"`{ast.unparse(node)}` subscripts something that is not a tensor")

    def slices(self, tensor: TensorRef, index: ast.expr, node: ast.AST) -> tuple[SliceExpr, ...]:
        items = index.elts if isinstance(index, ast.Tuple) else [index]
        slices: list[SliceExpr] = []
        for item in items:
            slices.append(self.one_slice(item, node))
        if len(slices) != tensor.type.rank:
            raise self.error(node, f"tensor `{tensor.name}` has {tensor.type.rank} axes, indexed with {len(slices)}")
        return tuple(slices)

    def one_slice(self, item: ast.expr, node: ast.AST) -> SliceExpr:
        if isinstance(item, ast.Slice):
            if item.step is not None:
                raise self.error(node, "tile slices have no step")
            return self.make_slice(item.lower, item.upper, node)
        if isinstance(item, ast.Call) and dotted(item.func) == "slice":
            if len(item.args) != 2:
                raise self.error(node, "`slice(start, stop)` takes two arguments")
            return self.make_slice(item.args[0], item.args[1], node)
        value = self.expr_or_value(item)
        if isinstance(value, SliceExpr):
            return value
        if isinstance(value, Expr) and not value.shape and (value.dtype.is_int or value.dtype == PY_INT):
            return SliceExpr(SliceType(1), self.scalar(value, node), squeeze=True, line=getattr(item, "lineno", 0))
        raise self.error(node, f"`{ast.unparse(item)}` is not a tile slice or an integer index")

    def make_slice(self, lower: ast.expr | None, upper: ast.expr | None, node: ast.AST) -> SliceExpr:
        """`lo : lo + C` or `C0 : C1`: the extent must be a compile-time constant."""
        if upper is None:
            raise self.error(node, "a tile slice needs an end: `lo : lo + C`")
        start = self.expr(lower) if lower is not None else Const(PY_INT, 0)
        stop = self.expr(upper)
        if isinstance(start, Const) and isinstance(stop, Const):
            extent = int(stop.value) - int(start.value)
        elif isinstance(upper, ast.BinOp) and isinstance(upper.op, ast.Add) and lower is not None and \
                ast.dump(upper.left) == ast.dump(lower) and isinstance(self.expr(upper.right), Const):
            extent = int(self.expr(upper.right).value)
        else:
            raise self.error(node, "a slice extent must be a compile-time constant (`lo : lo + C`)")
        if extent <= 0:
            raise self.error(node, f"a tile slice must have a positive extent, got {extent}")
        return SliceExpr(SliceType(extent), self.scalar(start, node), line=getattr(node, "lineno", 0))

    def call(self, node: ast.Call) -> object:
        func = node.func
        if isinstance(func, ast.Attribute):
            owner = dotted(func.value)
            if owner == "block" and "block" not in self.env:
                return self.block_call(func.attr, node)
            if dtype_name(func) is not None and dtype_name(func) not in ("int", "float", "bool") and \
                    not (isinstance(func.value, ast.Name) and func.value.id in self.env):
                return self.dtype_call(D.BY_NAME[dtype_name(func)], node)
            base = self.expr_or_value(func.value)
            if isinstance(base, Expr):
                return self.method(func.attr, base, node)
            raise self.error(node, f"`{ast.unparse(func)}` is not captured on the tile path")
        name = dotted(func)
        if name in self.env:
            raise self.error(node, f"`{name}` is not callable in a kernel")
        match name:
            case "zeros":
                return self.call_zeros(node)
            case "arange":
                return self.call_arange(node)
            case "where":
                return self.call_where(node)
            case "maximum" | "minimum":
                if len(node.args) != 2:
                    raise self.error(node, f"`{name}(a, b)` takes two tiles")
                return self.math(BINARY_MATH[name], [self.expr(a) for a in node.args], node)
            case "slice":  # `slice(stop)` or `slice(start, stop)` as a value (reference capture.py:2509-2510)
                if node.keywords or not 1 <= len(node.args) <= 2:
                    raise self.error(node, "`slice(start, stop)` takes one or two arguments")
                lower = node.args[0] if len(node.args) == 2 else None
                return self.make_slice(lower, node.args[-1], node)
        if dtype_name(func) is not None and dtype_name(func) not in ("int", "float", "bool"):
            return self.dtype_call(D.BY_NAME[dtype_name(func)], node)
        raise self.error(node, f"`{name}(...)` is not captured on the tile path")

    def block_call(self, attr: str, node: ast.Call) -> object:
        if attr == "index":
            return _BlockIndexValue()
        if attr == "tile":
            sizes = [int(self.constant(a, "a tile size")) for a in node.args]
            if node.keywords or not 1 <= len(sizes) <= 2:
                raise self.error(node, "`block.tile` takes one size (along x) or two (rows along y, columns along x)")
            axes = "yx"[-len(sizes):]
            tiles = tuple(
                SliceExpr(SliceType(size),
                          Binary(PY_INT, Op.MUL, BlockIndex(PY_INT, axis), Const(PY_INT, size)),
                          line=node.lineno)
                for axis, size in zip(axes, sizes)
            )
            return tiles[0] if len(tiles) == 1 else Packed(tiles)
        raise self.error(node, f"`block.{attr}` is not captured on the tile path")

    def dtype_call(self, dtype: Dtype, node: ast.Call) -> Expr:
        if len(node.args) != 1:
            raise self.error(node, f"`{dtype}(x)` converts one value")
        value = self.expr(node.args[0])
        if isinstance(value, Const):
            return Const(dtype, value.value, line=node.lineno)
        return self.cast(value, dtype)

    def call_zeros(self, node: ast.Call) -> Expr:
        if node.keywords:
            raise self.error(node, "`zeros(space=...)` is not lowered on the tile path")
        if not node.args or (dtype := dtype_name(node.args[0])) is None:
            raise self.error(node, "`zeros(dtype, *extent)` needs an element type first")
        shape = tuple(int(self.constant(a, "a tile extent")) for a in node.args[1:])
        if not shape or any(e <= 0 for e in shape):
            raise self.error(node, "a tile needs positive extents")
        return Zeros(TileType(D.BY_NAME[dtype], shape), line=node.lineno)

    def call_arange(self, node: ast.Call) -> Expr:
        """`arange(n, axis, rank=2, start=s)` (reference capture.py:2067-2079)."""
        args = dict(zip(("extent", "axis"), node.args))
        args |= {k.arg: k.value for k in node.keywords}
        if "extent" not in args:
            raise self.error(node, "`arange` needs an extent")
        extent = int(self.constant(args["extent"], "a tile extent"))
        axis = int(self.constant(args["axis"], "an axis")) if "axis" in args else 0
        rank = int(self.constant(args["rank"], "a rank")) if "rank" in args else 1
        if not 0 <= axis < rank:
            raise self.error(node, f"`arange` axis {axis} is out of range for rank {rank}")
        shape = tuple(extent if a == axis else 1 for a in range(rank))
        start = self.cast(self.expr(args["start"]), I32) if "start" in args else Const(I32, 0)
        return Arange(TileType(I32, shape), axis, start, line=node.lineno)

    def call_where(self, node: ast.Call) -> Expr:
        """`where(condition, x, y)` (reference capture.py:2046-2065)."""
        if len(node.args) != 3:
            raise self.error(node, "`where(condition, x, y)` takes three arguments")
        condition, x, y = (self.expr(a) for a in node.args)
        if condition.dtype != BOOL:
            raise self.error(node, f"`where` needs a bool condition, got {condition.type}; compare with <, > or ==")
        dtype = D.common(x.dtype, y.dtype)
        if dtype is None:
            raise self.error(node, f"`where` branches have types {x.type} and {y.type}; convert one with .to(...)")
        shape = self.broadcast(self.broadcast(condition.shape, x.shape, node), y.shape, node)
        x, y = self.coerce(x, dtype), self.coerce(y, dtype)
        kind = TileType(dtype, shape) if shape else dtype
        return Select(kind, condition, x, y, line=node.lineno)

    def tensor_dtype(self, node: ast.AST) -> Dtype | None:
        """The element type of `x.dtype` for a tensor parameter `x`, else None."""
        if isinstance(node, ast.Attribute) and node.attr == "dtype" and isinstance(node.value, ast.Name):
            for name, kind in self.params:
                if name == node.value.id and isinstance(kind, TensorType):
                    return kind.dtype
        return None

    def method(self, name: str, base: Expr, node: ast.Call) -> Expr:
        if name == "to":
            if len(node.args) == 1 and (element := self.tensor_dtype(node.args[0])) is not None:
                return self.cast(base, element)
            if len(node.args) != 1 or (dtype := dtype_name(node.args[0])) is None:
                raise self.error(node, "`.to(dtype)` takes one element type")
            return self.cast(base, D.BY_NAME[dtype])
        if name == "transpose":
            if node.args or node.keywords:
                raise self.error(node, "`transpose()` takes no arguments; a tile has two axes")
            if len(base.shape) != 2:
                raise self.error(node, f"`transpose()` needs a rank-2 tile, got {base.type}")
            return Transpose(TileType(base.dtype, base.shape[::-1]), base, line=node.lineno)
        if name in ARITHMETIC:
            return self.binary(ARITHMETIC[name], base, self.single(node), node)
        if name in BINARY_MATH:
            return self.math(BINARY_MATH[name], [base, self.single(node)], node)
        if name in UNARY_MATH:
            if node.args or node.keywords:
                raise self.error(node, f"`.{name}()` takes no arguments")
            return self.math(UNARY_MATH[name], [base], node)
        if name in ("max", "min", "sum"):
            return self.reduction(Reduction(name), base, node)
        if name in NORMALIZING or name in ("logsumexp", "norm"):
            return self.normalizing(name, base, node)
        raise self.error(node, f"`.{name}()` is not captured on the tile path")

    def normalizing(self, name: str, base: Expr, node: ast.Call) -> Expr:
        """`x.softmax(axis=1)`, `x.log_softmax(axis)`, `x.logsumexp(axis, keepdims)`, `x.norm(axis, keepdims)`:
        built from max, sum, exp, log and sqrt as the reference builds them (capture.py:2883-2917); softmax and
        log_softmax keep the shape, the default axis is the last."""
        names = ("axis",) if name in NORMALIZING else ("axis", "keepdims")
        args = dict(zip(names, node.args)) | {k.arg: k.value for k in node.keywords}
        if set(args) - set(names):
            raise self.error(node, f"`.{name}()` takes {' and '.join(names)}")
        axis = int(self.constant(args["axis"], "an axis")) if "axis" in args else -1
        keepdims = bool(self.constant(args["keepdims"], "keepdims")) if "keepdims" in args else False
        rank = len(base.shape)
        if not rank:
            raise self.error(node, f".{name}() reduces a tile, got {base.type}")
        if not -rank <= axis < rank:
            raise self.error(node, f"axis {axis} is out of range for a rank-{rank} tile")
        if not base.dtype.is_float:
            raise self.error(node, f".{name}() needs a float tile, got {base.type}")
        axis %= rank

        def reduce(op: Reduction, x: Expr, keep: bool) -> Expr:
            shape = x.shape[:axis] + ((1,) if keep else ()) + x.shape[axis + 1:]
            if not shape:
                raise self.error(node, "reducing a rank-1 tile to a scalar is not supported; pass keepdims=True")
            return Reduce(TileType(x.dtype, shape), op, x, axis, keep, line=node.lineno)

        def shifted() -> Expr:  # e^(x - max), the stable exponent shared by softmax and logsumexp
            return self.math(Fn.EXP, [self.binary(Op.SUB, base, reduce(Reduction.MAX, base, True), node)], node)

        if name == "softmax":
            return self.binary(Op.DIV, shifted(), reduce(Reduction.SUM, shifted(), True), node)
        if name == "log_softmax":
            top = reduce(Reduction.MAX, base, True)
            logsum = self.math(Fn.LOG, [reduce(Reduction.SUM, shifted(), True)], node)
            return self.binary(Op.SUB, base, self.binary(Op.ADD, logsum, top, node), node)
        if name == "logsumexp":
            top = reduce(Reduction.MAX, base, keepdims)
            return self.binary(Op.ADD, self.math(Fn.LOG, [reduce(Reduction.SUM, shifted(), keepdims)], node), top,
                               node)
        return self.math(Fn.SQRT, [reduce(Reduction.SUM, self.binary(Op.MUL, base, base, node), keepdims)], node)

    def single(self, node: ast.Call) -> Expr:
        if len(node.args) + len(node.keywords) != 1:
            raise self.error(node, "this operation takes one operand")
        return self.expr(node.args[0] if node.args else node.keywords[0].value)

    def reduction(self, op: Reduction, base: Expr, node: ast.Call) -> Expr:
        """`x.max(axis=1, keepdims=True)` (reference capture.py:2883-2927); the default axis is the last."""
        args = dict(zip(("axis", "keepdims"), node.args)) | {k.arg: k.value for k in node.keywords}
        if set(args) - {"axis", "keepdims"}:
            raise self.error(node, f"`.{op.value}()` takes axis and keepdims")
        axis = int(self.constant(args["axis"], "an axis")) if "axis" in args else -1
        keepdims = bool(self.constant(args["keepdims"], "keepdims")) if "keepdims" in args else False
        rank = len(base.shape)
        if not rank:
            raise self.error(node, f".{op.value}() reduces a tile, got {base.type}")
        if not -rank <= axis < rank:
            raise self.error(node, f"axis {axis} is out of range for a rank-{rank} tile")
        axis %= rank
        shape = base.shape[:axis] + ((1,) if keepdims else ()) + base.shape[axis + 1:]
        if not shape:
            raise self.error(node, "reducing a rank-1 tile to a scalar is not supported; pass keepdims=True")
        return Reduce(TileType(base.dtype, shape), op, base, axis, keepdims, line=node.lineno)

    # ---- typing

    def constant(self, node: ast.expr, what: str) -> int | float | bool:
        value = self.expr(node)
        if not isinstance(value, Const):
            raise self.error(node, f"{what} must be a compile-time constant")
        return value.value

    def broadcast(self, a: tuple[int, ...], b: tuple[int, ...], node: ast.AST) -> tuple[int, ...]:
        """numpy broadcasting of tile shapes, aligned from the right (reference compiler/capture.py:1531-1541)."""
        if not a or not b:
            return a or b
        width = max(len(a), len(b))
        a, b = (1,) * (width - len(a)) + a, (1,) * (width - len(b)) + b
        out = []
        for x, y in zip(a, b):
            if x != y and 1 not in (x, y):
                raise self.error(node, f"tile shapes {list(a)} and {list(b)} do not broadcast")
            out.append(max(x, y))
        return tuple(out)

    def coerce(self, value: Expr, dtype: Dtype) -> Expr:
        if value.dtype == dtype:
            return value
        if isinstance(value, Const):
            converted = bool(value.value) if dtype == BOOL else (
                float(value.value) if dtype.is_float or dtype == PY_FLOAT else int(value.value))
            return Const(dtype, converted, line=value.line)
        return self.cast(value, dtype)

    def cast(self, value: Expr, dtype: Dtype) -> Expr:
        if value.dtype == dtype:
            return value
        kind = TileType(dtype, value.shape) if value.shape else dtype
        return Cast(kind, value, line=value.line)

    def scalar(self, value: Expr, node: ast.AST) -> Expr:
        if value.shape:
            raise self.error(node, "a loop bound or slice start is a scalar")
        if not (value.dtype.is_int or value.dtype == PY_INT):
            raise self.error(node, f"a loop bound or slice start is an integer, got {value.dtype}")
        return value

    def binary(self, op: Op, lhs: Expr, rhs: Expr, node: ast.AST) -> Expr:
        if isinstance(lhs, Const) and isinstance(rhs, Const) and lhs.dtype.is_py and rhs.dtype.is_py:
            return self.fold(op, lhs, rhs, node)
        dtype = D.common(lhs.dtype, rhs.dtype)
        if dtype is None:
            raise self.error(node, f"dtype mismatch in `{op.value}`: {lhs.dtype} and {rhs.dtype}; convert one side "
                             "with .to(...)")
        if dtype == PY_FLOAT and (lhs.shape or rhs.shape):
            dtype = F32
        shape = self.broadcast(lhs.shape, rhs.shape, node)
        lhs, rhs = self.coerce(lhs, dtype), self.coerce(rhs, dtype)
        result = BOOL if op in (*COMPARISONS,) else dtype
        if op in (Op.AND, Op.OR) and dtype != BOOL:
            raise self.error(node, "`&` and `|` combine bool tiles")
        kind = TileType(result, shape) if shape else result
        return Binary(kind, op, lhs, rhs, line=getattr(node, "lineno", 0))

    def fold(self, op: Op, lhs: Const, rhs: Const, node: ast.AST) -> Const:
        a, b = lhs.value, rhs.value
        integer = lhs.dtype == PY_INT and rhs.dtype == PY_INT
        match op:
            case Op.ADD: value = a + b
            case Op.SUB: value = a - b
            case Op.MUL: value = a * b
            case Op.DIV: value = a / b
            case Op.MOD: value = a % b
            case Op.LT: value = a < b
            case Op.LE: value = a <= b
            case Op.GT: value = a > b
            case Op.GE: value = a >= b
            case Op.EQ: value = a == b
            case Op.NE: value = a != b
            case _: raise self.error(node, f"`{op.value}` on constants")
        if isinstance(value, bool):
            return Const(BOOL, value)
        return Const(PY_INT if integer and op is not Op.DIV else PY_FLOAT, value)

    def math(self, fn: Fn, operands: list[Expr], node: ast.AST) -> Expr:
        dtype = operands[0].dtype
        for operand in operands[1:]:
            common = D.common(dtype, operand.dtype)
            if common is None:
                raise self.error(node, f"dtype mismatch in `{fn.value}`: "
                                 f"{', '.join(str(o.dtype) for o in operands)}; convert one side with .to(...)")
            dtype = common
        if dtype == PY_FLOAT:
            dtype = F32
        if dtype not in (D.F32, D.F64) and not (fn in BINARY_MATH.values() and (dtype.is_int or dtype.is_float)):
            raise self.error(node, f"{fn.value} needs f32 or f64, got {dtype}; convert with .to(T.f32)")
        shape: tuple[int, ...] = ()
        for operand in operands:
            shape = self.broadcast(shape, operand.shape, node)
        args = tuple(self.coerce(o, dtype) for o in operands)
        return Math(TileType(dtype, shape) if shape else dtype, fn, args, line=getattr(node, "lineno", 0))


def capture(path: str | Path, name: str, consts: dict | None = None, dtypes: dict | None = None) -> Kernel:
    """The IR of kernel `name` in `path`, specialized on the `Const` values in `consts` ({param: {field: value}})
    and the element types in `dtypes` ({param: Dtype}), which override the annotations."""
    path = Path(path)
    source = path.read_text()
    module = ast.parse(source, filename=str(path))
    fn = next((n for n in module.body if isinstance(n, ast.FunctionDef) and n.name == name), None)
    if fn is None:
        raise CaptureError(f"{path}: no function `{name}`")
    capture_ = Capture(path, source, fn, consts or {}, dtypes or {}, struct_defaults(module))
    capture_.parameters()
    body = capture_.block(fn.body)
    space = tuple((axis, size, tuple(extents)) for axis, (size, extents) in sorted(capture_.space.items()))
    frozen = tuple(
        (k, tuple(sorted(v.values.items()))) for k, v in capture_.env.items() if isinstance(v, Config)
    )
    signature = tuple(a.arg for a in fn.args.args)
    return Kernel(name, tuple(capture_.params), tuple(capture_.tiles), body, space, frozen, str(path), signature)

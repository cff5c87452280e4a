"""Symbolic dataflow of a captured tile program, for recognising what a program computes rather than how it is
spelled.

`evaluate` runs the program's statements symbolically. A value is a nested tuple over the program's inputs:
parameters, tile loads, block indices, constants. Local variables and temporaries are substituted away, and the
operands of commutative operations (`+`, `*`, `maximum`, `minimum`, `==`, `!=`) are put in one order. Constant tiles
are folded (`zeros(...) - 1e30` is the tile filled with -1e30), and so are `x + 0`, `x * 1` and comparisons written
the other way round (`a >= b` is `b <= a`). A `for` loop is evaluated once with every variable it re-assigns bound
to a `("state", name)` symbol: the loop's effect is then one update expression per carried variable, over the
state symbols, the loop variable and what the loop reads. Two programs that compute the same values in the same
float32 operations (up to the order of commutative operands) get equal expressions, whatever their variable names,
statement order or temporaries.

This is the recognition the reference does not need: its compiler lowers every program through one generic path
(src/krn/compiler/emit.py:924-955); this backend maps whole programs onto hand-written kernels and uses the
dataflow to decide that a program is one of them.
"""

from dataclasses import dataclass, field

from krn_amd.compiler import ir

COMMUTATIVE = {ir.Op.ADD, ir.Op.MUL, ir.Op.EQ, ir.Op.NE, ir.Op.AND, ir.Op.OR}
FLIPPED = {ir.Op.GE: ir.Op.LE, ir.Op.GT: ir.Op.LT}  # a >= b is b <= a


class Unsupported(Exception):
    """The program uses a construct the dataflow does not model (the caller then does not recognise it)."""


@dataclass
class Loop:
    """One evaluated `for` loop: its variable, bounds and step, and the initial value and the update (one
    iteration's new value, over the state symbols) of each variable it carries."""

    var: str
    lo: tuple
    hi: tuple
    step: int
    init: dict[str, tuple] = field(default_factory=dict)
    update: dict[str, tuple] = field(default_factory=dict)


@dataclass
class Dataflow:
    """The evaluated program: its loops in order and its stores as (tensor, slices, value)."""

    loops: list[Loop] = field(default_factory=list)
    stores: list[tuple[str, tuple, tuple]] = field(default_factory=list)


def _key(value: tuple) -> str:
    return repr(value)


def _sorted(a: tuple, b: tuple) -> tuple[tuple, tuple]:
    return (a, b) if _key(a) <= _key(b) else (b, a)


def _fill_value(value: tuple):
    """The element of a constant tile or scalar constant, else None."""
    if value[0] == "const":
        return value[1]
    if value[0] == "fill":
        return value[1]
    return None


class Evaluator:
    def __init__(self) -> None:
        self.flow = Dataflow()

    # expressions
    def expr(self, e: ir.Expr, env: dict) -> tuple:
        match e:
            case ir.Const(value=v):
                return ("const", float(v) if isinstance(v, (int, float)) and not isinstance(v, bool) else v)
            case ir.Param(name=n):
                return ("param", n)
            case ir.Var(name=n):
                if n not in env:
                    raise Unsupported(f"variable {n} read before assignment")
                return env[n]
            case ir.Dim(tensor=t, axis=a):
                return ("dim", t.name, a)
            case ir.BlockIndex(axis=a):
                return ("block", a)
            case ir.Zeros(type=t):
                return ("fill", 0.0, t.shape)
            case ir.Unary(op=ir.Op.NEG, operand=o):
                x = self.expr(o, env)
                f = _fill_value(x)
                if f is not None and not isinstance(f, bool):
                    return ("const", -f) if x[0] == "const" else ("fill", -f, x[2])
                return ("neg", x)
            case ir.Binary(op=op, lhs=a, rhs=b):
                return self.binary(op, self.expr(a, env), self.expr(b, env), e)
            case ir.Math(fn=fn, args=args):
                xs = tuple(self.expr(a, env) for a in args)
                if fn in (ir.Fn.MAXIMUM, ir.Fn.MINIMUM):
                    xs = _sorted(*xs)
                return ("math", fn.value, *xs)
            case ir.Reduce(op=op, operand=o, axis=axis, keepdims=keep):
                return ("reduce", op.value, axis, keep, self.expr(o, env))
            case ir.Cast(operand=o, type=t):
                x = self.expr(o, env)
                dtype = t.dtype if isinstance(t, ir.TileType) else t
                if x[0] == "cast" and x[1] == dtype:
                    return x
                return ("cast", dtype, x)
            case ir.Select(cond=c, then=a, orelse=b):
                cond = self.expr(c, env)
                then, orelse = self.expr(a, env), self.expr(b, env)
                if cond[0] == "bin" and cond[1] == ir.Op.LT.value:  # where(a < b, x, y) is where(b <= a, y, x)
                    cond, then, orelse = ("bin", ir.Op.LE.value, cond[3], cond[2]), orelse, then
                return ("select", cond, then, orelse)
            case ir.Transpose(operand=o):
                return ("transpose", self.expr(o, env))
            case ir.Arange(axis=axis, start=s, type=t):
                return ("arange", axis, t.shape, self.expr(s, env))
            case ir.TileLoad(tensor=t, slices=slices):
                return ("load", t.name, tuple(self.slice(s, env) for s in slices))
        raise Unsupported(f"{type(e).__name__} is not modelled")

    def slice(self, s: ir.SliceExpr, env: dict) -> tuple:
        return (self.expr(s.start, env), s.extent, s.squeeze)

    def binary(self, op: ir.Op, a: tuple, b: tuple, node: ir.Binary) -> tuple:
        fa, fb = _fill_value(a), _fill_value(b)
        tile = node.shape
        if fa is not None and fb is not None and not isinstance(fa, bool) and not isinstance(fb, bool):
            value = {ir.Op.ADD: lambda: fa + fb, ir.Op.SUB: lambda: fa - fb, ir.Op.MUL: lambda: fa * fb}.get(op)
            if value is not None:
                return ("fill", value(), tile) if tile else ("const", value())
        if op == ir.Op.ADD and fb == 0.0 and b[0] == "fill":
            return a
        if op == ir.Op.ADD and fa == 0.0 and a[0] == "fill":
            return b
        if op == ir.Op.MUL and fb == 1.0 and b[0] == "const":
            return a
        if op == ir.Op.MUL and fa == 1.0 and a[0] == "const":
            return b
        if op in FLIPPED:
            op, a, b = FLIPPED[op], b, a
        if op in COMMUTATIVE:
            a, b = _sorted(a, b)
        return ("bin", op.value, a, b)

    # statements
    def block(self, body: tuple, env: dict) -> None:
        for s in body:
            self.statement(s, env)

    def statement(self, s: ir.Stmt, env: dict) -> None:
        match s:
            case ir.TileAssign(var=v, value=e) | ir.Assign(var=v, value=e):
                env[v.name] = self.expr(e, env)
            case ir.Accumulate(acc=acc, lhs=a, rhs=b):
                product = ("matmul", self.expr(a, env), self.expr(b, env))
                env[acc.name] = self.binary(ir.Op.ADD, env[acc.name], product, ir.Binary(
                    acc.type, ir.Op.ADD, acc, acc)) if acc.name in env else product
            case ir.TileStore(tensor=t, slices=slices, value=e):
                self.flow.stores.append((t.name, tuple(self.slice(x, env) for x in slices), self.expr(e, env)))
            case ir.If(cond=ir.Const(value=c), then=then, orelse=orelse):
                self.block(then if c else orelse, env)
            case ir.For(var=v, lo=lo, hi=hi, step=step, body=body):
                self.loop(v, lo, hi, step, body, env)
            case _:
                raise Unsupported(f"{type(s).__name__} is not modelled")

    def loop(self, var: ir.Var, lo: ir.Expr, hi: ir.Expr, step: int, body: tuple, env: dict) -> None:
        assigned = _assigned(body)
        carried = [n for n in assigned if n in env]
        loop = Loop(var.name, self.expr(lo, env), self.expr(hi, env), step,
                    init={n: env[n] for n in carried})
        inner = dict(env)
        for n in carried:
            inner[n] = ("state", n)
        inner[var.name] = ("loopvar", var.name)
        self.block(body, inner)
        loop.update = {n: inner[n] for n in carried}
        self.flow.loops.append(loop)
        for n in carried:  # after the loop a carried variable holds the loop's final state
            env[n] = ("final", n)
        for n in assigned:
            if n not in carried:
                env.pop(n, None)  # a loop-local value is not defined after a loop that may not run


def _assigned(body: tuple) -> list[str]:
    names: list[str] = []
    for s in body:
        match s:
            case ir.TileAssign(var=v) | ir.Assign(var=v) | ir.Accumulate(acc=v):
                if v.name not in names:
                    names.append(v.name)
            case ir.If(then=then, orelse=orelse):
                names += [n for n in _assigned(then) + _assigned(orelse) if n not in names]
            case ir.For(body=inner):
                names += [n for n in _assigned(inner) if n not in names]
    return names


def evaluate(kernel: ir.Kernel) -> Dataflow:
    """The program's dataflow; raises Unsupported for constructs outside the model."""
    evaluator = Evaluator()
    evaluator.block(kernel.body, {})
    return evaluator.flow


def scalar_value(value: tuple, params: dict):
    """A scalar value of the dataflow (constants, parameters and `+ - * /` over them) for these arguments, with each
    operation rounded to float32 as the program computes it; None when `value` is not such a scalar."""
    import numpy as np

    match value:
        case ("const", v) if not isinstance(v, bool):
            return np.float32(v)
        case ("param", n) if n in params:
            return np.float32(params[n])
        case ("cast", _, x):
            return scalar_value(x, params)
        case ("bin", op, a, b) if op in ("+", "-", "*", "/"):
            x, y = scalar_value(a, params), scalar_value(b, params)
            if x is None or y is None:
                return None
            with np.errstate(all="ignore"):
                return np.float32({"+": np.add, "-": np.subtract, "*": np.multiply, "/": np.divide}[op](x, y))
    return None


def is_scalar(value: tuple) -> bool:
    match value:
        case ("const", v):
            return not isinstance(v, bool)
        case ("param", _):
            return True
        case ("cast", _, x):
            return is_scalar(x)
        case ("bin", op, a, b) if op in ("+", "-", "*", "/"):
            return is_scalar(a) and is_scalar(b)
    return False

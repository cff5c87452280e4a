"""The CDNA4 (gfx950) lowering of captured tile programs: recognise the contraction programs the hand-written MFMA
kernels serve, and lower everything else through the generic HIP emitter.

What `lower` returns is a plan the HIP backend launches:

* `GemmPlan`: `acc = zeros(...)`, one K loop of `acc += a[rows, ks] @ b[cols, ks].transpose()` (or `b[ks, cols]`),
  and one store of an epilogue of `acc` into `c[rows, cols]` (after any `acc = f(acc)` steps) -> `krn_gemm_nt` with
  bf16/f16 (32x32x16 MFMA), fp8 e4m3 (32x32x64 f8f6f4 MFMA) or int8 (32x32x32 i8 MFMA) operands. The epilogue may
  multiply or add float32 scalars, per-row vectors (`s[rows, 0:1]`) and per-column vectors (`s[0:1, cols]`, or a
  bias `v[cols]` of f32/f16/bf16), and apply relu, gelu or silu, in the program's order, each rounded to float32,
  then convert to bf16/f16/f32 (or keep int32). The kernel picks its own tile sizes for 256 CUs;
  the program's `bm, bn, bk` change only the grid it asks for, which must cover the output.
* `AttentionPlan`: krn's flash-attention tile program (reference examples/04_libraries/08_flash_attention.py:35-59)
  with head dimension 64 or 128, f16 or bf16, causal or not -> `krn_attention_fwd`.
* `SoftmaxPlan`: krn's row-softmax programs, the long-row running form (reference examples/02_tiles_and_types/
  01_softmax_rows.py:27-40) and the one-tile forms (tests/helpers/example_softmax.py:12-24), f16, bf16 or f32
  -> `krn_softmax_rows`.
* `GenericPlan`: any other tile program -> hipgen (HIP C++ compiled by hiprtc).

Replaces the reference's compile-checked HIP renderer (src/krn/compiler/hip.py:20-183), which emitted 16x16x16
f16/bf16 MFMA only, refused fp8 (compiler/matrix.py:129-139) and had no int8 product.
"""

import dataclasses
import math
from dataclasses import dataclass, field

from krn_amd.compiler import ir
from krn_amd.dtypes import BF16, F8E4M3, F16, F32, I8, I32, Dtype

GEMM_OPERANDS = (BF16, F16, F8E4M3, I8)
ACTIVATIONS = {ir.Fn.RELU: "relu", ir.Fn.GELU: "gelu", ir.Fn.SILU: "silu"}


@dataclass(frozen=True)
class EpilogueOp:
    """One elementwise step after the product: `op` is "mul" or "add" with a scalar expression or a row/column vector
    read from `tensor` (shape (M, 1), (1, N) or (N,)), or the activation "relu", "gelu" or "silu"."""

    op: str
    scalar: ir.Expr | None = None
    tensor: str | None = None
    axis: str = ""  # "row" or "col" for a vector


@dataclass(frozen=True)
class GemmPlan:
    a: str
    b: str
    c: str
    layout: str  # "nt": b is (N, K); "nn": b is (K, N)
    operand: Dtype
    output: Dtype
    ops: tuple[EpilogueOp, ...]
    bm: int
    bn: int
    bk: int
    loop_extent: ir.Expr


@dataclass(frozen=True)
class AttentionPlan:
    q: str
    k: str
    v: str
    o: str
    scale: tuple  # the dataflow of the scalar the scores are multiplied by (dataflow.scalar_value evaluates it)
    dtype: Dtype
    d: int
    bq: int
    causal: bool
    base: float = 1.0  # the exponent's base as a power of 2: 1 for exp2, log2(e) for exp
    rank: int = 3  # 3: (heads, seq, d); 4: (batch, heads, seq, d)


@dataclass(frozen=True)
class SoftmaxPlan:
    x: str
    y: str
    dtype: Dtype
    rows: int  # rows per block of the program's grid
    cols: int  # the one-tile forms' column extent; the long-row form reads every column
    long_rows: bool


@dataclass
class GenericPlan:
    kernel: ir.Kernel
    source: str = ""
    shared: int = 0
    cache: dict = field(default_factory=dict)


def _block_slice(s: ir.SliceExpr, axis: str) -> int | None:
    """The tile size when `s` is `block.tile`'s slice along grid axis `axis`, else None."""
    match s:
        case ir.SliceExpr(start=ir.Binary(op=ir.Op.MUL, lhs=ir.BlockIndex(axis=a), rhs=ir.Const(value=size)),
                          squeeze=False) if a == axis:
            return int(size)
    return None


def _k_slice(s: ir.SliceExpr, var: ir.Var, bk: int) -> bool:
    return isinstance(s.start, ir.Var) and s.start == var and s.extent == bk and not s.squeeze


def _substitute(e, var: ir.Var, value: ir.Expr):
    """`e` with every use of the tile variable `var` replaced by `value`."""
    if e == var:
        return value
    if not dataclasses.is_dataclass(e) or isinstance(e, type):
        return e
    changes = {}
    for f in dataclasses.fields(e):
        old = getattr(e, f.name)
        if isinstance(old, tuple):
            new = tuple(_substitute(x, var, value) for x in old)
        elif dataclasses.is_dataclass(old) and not isinstance(old, type):
            new = _substitute(old, var, value)
        else:
            continue
        if new is not old and new != old:
            changes[f.name] = new
    return dataclasses.replace(e, **changes) if changes else e


def match_gemm(kernel: ir.Kernel) -> GemmPlan | None:
    body = kernel.body
    if len(body) < 3:
        return None
    init, loop, *post, store = body
    # `acc = f(acc)` steps after the loop (bias, activations) fold into the stored expression
    for statement in post:
        if not (isinstance(statement, ir.TileAssign) and isinstance(init, ir.TileAssign) and
                statement.var == init.var):
            return None
    if post and isinstance(store, ir.TileStore):
        value = init.var
        for statement in post:
            value = _substitute(statement.value, init.var, value)
        store = dataclasses.replace(store, value=_substitute(store.value, init.var, value))
    if not (isinstance(init, ir.TileAssign) and isinstance(init.value, ir.Zeros)):
        return None
    acc = init.var
    if acc.dtype not in (F32, I32) or len(acc.shape) != 2:
        return None
    bm, bn = acc.shape
    if not (isinstance(loop, ir.For) and len(loop.body) == 1 and isinstance(loop.body[0], ir.Accumulate)):
        return None
    if not (isinstance(loop.lo, ir.Const) and loop.lo.value == 0):
        return None
    step = loop.body[0]
    if step.acc != acc:
        return None
    bk = loop.step
    lhs, rhs = step.lhs, step.rhs
    # A: a[rows, ks]
    if not (isinstance(lhs, ir.TileLoad) and lhs.tensor.type.rank == 2):
        return None
    if _block_slice(lhs.slices[0], "y") != bm or not _k_slice(lhs.slices[1], loop.var, bk):
        return None
    # B: b[cols, ks].transpose() or b[ks, cols]
    if isinstance(rhs, ir.Transpose) and isinstance(rhs.operand, ir.TileLoad) and rhs.operand.tensor.type.rank == 2:
        load, layout = rhs.operand, "nt"
        if _block_slice(load.slices[0], "x") != bn or not _k_slice(load.slices[1], loop.var, bk):
            return None
    elif isinstance(rhs, ir.TileLoad) and rhs.tensor.type.rank == 2:
        load, layout = rhs, "nn"
        if not _k_slice(load.slices[0], loop.var, bk) or _block_slice(load.slices[1], "x") != bn:
            return None
    else:
        return None
    operand = lhs.dtype
    if operand != load.dtype or operand not in GEMM_OPERANDS or layout == "nn" and operand not in (BF16, F16):
        return None
    if (operand == I8) != (acc.dtype == I32):
        return None
    # C: c[rows, cols] = epilogue(acc)
    if not (isinstance(store, ir.TileStore) and store.tensor.type.rank == 2):
        return None
    if _block_slice(store.slices[0], "y") != bm or _block_slice(store.slices[1], "x") != bn:
        return None
    value, output = store.value, store.tensor.type.dtype
    if output not in (F32, F16, BF16, I32):
        return None
    if output == I32:
        if value != acc or acc.dtype != I32:
            return None
        ops: list[EpilogueOp] | None = []
    else:
        if isinstance(value, ir.Cast) and value.dtype == output and output != F32:
            value = value.operand
        ops = _epilogue(value, acc, bm, bn)
        if ops is None:
            return None
    return GemmPlan(lhs.tensor.name, load.tensor.name, store.tensor.name, layout, operand, output, tuple(ops), bm, bn,
                    bk, loop.hi)


def _epilogue(e: ir.Expr, acc: ir.Var, bm: int, bn: int) -> list[EpilogueOp] | None:
    """The chain of float32 operations from `acc` to `e`, innermost first; None when `e` is not such a chain."""
    if e == acc:
        return [] if acc.dtype == F32 else None
    if isinstance(e, ir.Cast) and e.operand == acc and acc.dtype == I32 and e.dtype == F32:
        return []
    if isinstance(e, ir.Math) and e.fn in ACTIVATIONS and e.dtype == F32 and len(e.args) == 1:
        chain = _epilogue(e.args[0], acc, bm, bn)
        return None if chain is None else [*chain, EpilogueOp(ACTIVATIONS[e.fn])]
    if isinstance(e, ir.Binary) and e.op in (ir.Op.MUL, ir.Op.ADD) and e.dtype == F32:
        for inner, other in ((e.lhs, e.rhs), (e.rhs, e.lhs)):
            chain = _epilogue(inner, acc, bm, bn)
            if chain is None:
                continue
            operand = _operand(other, bm, bn)
            if operand is None:
                continue
            name = "mul" if e.op is ir.Op.MUL else "add"
            return [*chain, EpilogueOp(name, *operand)]
    return None


def _operand(e: ir.Expr, bm: int, bn: int) -> tuple | None:
    """A scalar float32 expression over parameters and constants, or a row/column vector tile load: a (bm, 1) or
    (1, bn) slice of a float32 matrix, or the `v[cols]` slice of a float32/f16/bf16 vector widened to float32."""
    if not e.shape:
        if _scalar_expr(e) and e.dtype == F32:
            return (e, None, "")
        return None
    vector = e.operand if isinstance(e, ir.Cast) and e.dtype == F32 else e
    if isinstance(vector, ir.TileLoad) and vector.tensor.type.rank == 1 and vector.shape == (bn,) and \
            vector.dtype in (F32, F16, BF16) and _block_slice(vector.slices[0], "x") == bn:
        return (None, vector.tensor.name, "col")
    if isinstance(e, ir.TileLoad) and e.dtype == F32 and e.tensor.type.rank == 2 and len(e.shape) == 2:
        rows, cols = e.slices
        if e.shape == (bm, 1) and _block_slice(rows, "y") == bm and isinstance(cols.start, ir.Const) and \
                cols.start.value == 0 and cols.extent == 1:
            return (None, e.tensor.name, "row")
        if e.shape == (1, bn) and _block_slice(cols, "x") == bn and isinstance(rows.start, ir.Const) and \
                rows.start.value == 0 and rows.extent == 1:
            return (None, e.tensor.name, "col")
    return None


def _scalar_expr(e: ir.Expr) -> bool:
    match e:
        case ir.Const() | ir.Param():
            return True
        case ir.Binary(op=op, lhs=a, rhs=b) if op in (ir.Op.MUL, ir.Op.ADD, ir.Op.SUB, ir.Op.DIV):
            return _scalar_expr(a) and _scalar_expr(b)
        case ir.Cast(operand=o):
            return _scalar_expr(o)
    return False


def _strip_cast(x: tuple) -> tuple:
    return x[2] if x[0] == "cast" else x


def _const(x: tuple, value: float) -> bool:
    return x[0] == "const" and x[1] == value


def _masked_value(x: tuple) -> bool:
    """A constant at or below -1e30 (or -inf): exp2 of it minus any finite row maximum is 0."""
    return x[0] in ("const", "fill") and not isinstance(x[1], bool) and x[1] <= -1.0e30


def match_attention(kernel: ir.Kernel) -> AttentionPlan | None:
    """krn's flash-attention program (reference examples/04_libraries/08_flash_attention.py:35-59), recognised by
    what it computes: one loop over key tiles `c` of a key or value tensor's sequence axis, carrying a running row
    maximum `m`, row sum `l` and output `acc` started at (<= -1e30, 0, 0), with one iteration

        s = scale * (Q @ K[c:c+bk].T)             (scale: a scalar expression; optionally masked to <= -1e30 where
                                                   k_pos > q_pos, k_pos = c + arange(bk), q_pos = rows + arange(bq))
        m' = maximum(m, rowmax(s)),  p = exp2(s - m'),  corr = exp2(m - m')
        l' = l * corr + rowsum(p),   acc' = acc * corr + p.to(dtype) @ V[c:c+bk]

    (or exp in place of both exp2, which is exp2 with the scale times log2(e)), and one store `o[rows] = (acc /
    l).to(dtype)`; Q, K, V and O are (heads, seq, d) tensors indexed by block y, or (batch, heads, seq, d) indexed
    by blocks z and y, with the query rows `block.tile(bq)` along x. Names, temporaries, statement order, operand
    order of commutative operations and the tiling (bq, bk) are free. The dataflow is compared, not the spelling."""
    from krn_amd.compiler import dataflow as df

    tensors = [(n, t) for n, t in kernel.params if isinstance(t, ir.TensorType)]
    if len(tensors) != 4 or len({t.rank for _, t in tensors}) != 1 or tensors[0][1].rank not in (3, 4):
        return None
    rank = tensors[0][1].rank
    dtype = tensors[0][1].dtype
    if dtype not in (F16, BF16) or any(t.dtype != dtype for _, t in tensors):
        return None
    try:
        flow = df.evaluate(kernel)
    except (df.Unsupported, KeyError, IndexError, TypeError):
        return None
    if len(flow.loops) != 1 or len(flow.stores) != 1:
        return None
    loop, (o_name, o_slices, stored) = flow.loops[0], flow.stores[0]
    heads = (((("block", "y"), 1, True),) if rank == 3 else ((("block", "z"), 1, True), (("block", "y"), 1, True)))
    # the store: o[heads, rows, 0:d] = (acc / l).to(dtype)
    if not (stored[0] == "cast" and stored[1] == dtype and stored[2][0] == "bin" and stored[2][1] == "/"):
        return None
    acc_f, l_f = stored[2][2], stored[2][3]
    if acc_f[0] != "final" or l_f[0] != "final":
        return None
    acc, l = acc_f[1], l_f[1]
    if len(o_slices) != rank or o_slices[:-2] != heads:
        return None
    rows, d_slice = o_slices[-2], o_slices[-1]
    bq, d = rows[1], d_slice[1]
    if rows[2] or rows[0] != ("bin", "*", *sorted((("block", "x"), ("const", float(bq))), key=repr)):
        return None
    if d_slice != (("const", 0.0), d, False) or d not in (64, 128):
        return None
    carried = set(loop.init)
    if not {acc, l} <= carried or len(carried) != 3:
        return None
    (m,) = carried - {acc, l}
    # initial values
    if loop.init[acc] != ("fill", 0.0, (bq, d)) or loop.init[l] != ("fill", 0.0, (bq, 1)):
        return None
    if not (_masked_value(loop.init[m]) and (loop.init[m][0] == "const" or loop.init[m][2] == (bq, 1))):
        return None
    # m' = maximum(m, rowmax(s))
    m_new = loop.update[m]
    if not (m_new[0] == "math" and m_new[1] == "maximum" and ("state", m) in m_new[2:]):
        return None
    rowmax = m_new[3] if m_new[2] == ("state", m) else m_new[2]
    if not (rowmax[0] == "reduce" and rowmax[1:4] == ("max", 1, True)):
        return None
    s = rowmax[4]
    # l' = l * corr + rowsum(p);  acc' = acc * corr + p.to(dtype) @ V
    def split(update: tuple, state: str) -> tuple[tuple, tuple] | None:
        if not (update[0] == "bin" and update[1] == "+"):
            return None
        for scaled, other in ((update[2], update[3]), (update[3], update[2])):
            if scaled[0] == "bin" and scaled[1] == "*" and ("state", state) in scaled[2:]:
                corr = scaled[3] if scaled[2] == ("state", state) else scaled[2]
                return corr, other
        return None
    l_parts, acc_parts = split(loop.update[l], l), split(loop.update[acc], acc)
    if l_parts is None or acc_parts is None or l_parts[0] != acc_parts[0]:
        return None
    corr, rowsum = l_parts
    fn = corr[1] if corr[0] == "math" else None
    if fn not in ("exp2", "exp") or corr[2] != ("bin", "-", ("state", m), m_new):
        return None
    p = ("math", fn, ("bin", "-", s, m_new))
    if rowsum != ("reduce", "sum", 1, True, p):
        return None
    pv = acc_parts[1]
    if not (pv[0] == "matmul" and pv[1] == ("cast", dtype, p) and pv[2][0] == "load"):
        return None
    v_load = pv[2]
    # s = scale * (Q @ K.T), optionally masked
    causal = False
    if s[0] == "select":
        cond, s0, masked = s[1], s[2], s[3]
        if not _masked_value(masked):
            return None
        # k_pos <= q_pos: arange along keys from the loop variable, along rows from the rows' start
        if not (cond[0] == "bin" and cond[1] == "<="):
            return None
        k_pos, q_pos = cond[2], cond[3]
        if not (k_pos[0] == "arange" and k_pos[1] == 1 and _strip_cast(k_pos[3]) == ("loopvar", loop.var)):
            return None
        if not (q_pos[0] == "arange" and q_pos[1] == 0 and q_pos[2] == (bq, 1) and _strip_cast(q_pos[3]) == rows[0]):
            return None
        causal = True
        s = s0
    if not (s[0] == "bin" and s[1] == "*"):
        return None
    product = next((x for x in s[2:] if x[0] == "matmul"), None)
    scale = s[2] if s[3] is product else s[3]
    if product is None or not df.is_scalar(scale):
        return None
    q_load, kt = product[1], product[2]
    if not (q_load[0] == "load" and kt[0] == "transpose" and kt[1][0] == "load"):
        return None
    k_load = kt[1]
    if q_load[2] != (*heads, rows, d_slice):
        return None
    bk = k_load[2][-2][1]
    if bk != loop.step or not _const(loop.lo, 0.0):
        return None
    key_slices = (*heads, (("loopvar", loop.var), bk, False), d_slice)
    if k_load[2] != key_slices or v_load[2] != key_slices:
        return None
    names = {q_load[1], k_load[1], v_load[1], o_name}
    if len(names) != 4 or loop.hi not in (("dim", k_load[1], rank - 2), ("dim", v_load[1], rank - 2)):
        return None
    return AttentionPlan(q_load[1], k_load[1], v_load[1], o_name, scale, dtype, int(d), int(bq), causal,
                         1.0 if fn == "exp2" else math.log2(math.e), rank)


def match_softmax(kernel: ir.Kernel) -> SoftmaxPlan | None:
    """krn's row softmax, recognised by what it computes over x and y of one element type (f16, bf16 or f32, math in
    float32), with R = `block.tile(R)` rows per block along x:

    * one tile of C columns (reference tests/helpers/example_softmax.py:12-24, `.softmax(axis=1)` or its steps):
      `y[rows, 0:C] = (e / rowsum(e)).to(dtype)` with `e = exp(v - rowmax(v))`, `v = x[rows, 0:C].to(f32)`;
    * long rows (reference examples/02_tiles_and_types/01_softmax_rows.py:27-40): a loop over column chunks of x's
      width carrying a running maximum m (from a constant at or below -3e38) and sum s (from 0), `m' = maximum(m,
      rowmax(v))`, `s' = s * exp(m - m') + rowsum(exp(v - m'))`, then a loop over the same chunks storing
      `(exp(v - m) / s).to(dtype)`.

    Names, temporaries and operand order are free; the dataflow is compared, not the spelling."""
    from krn_amd.compiler import dataflow as df

    tensors = [(n, t) for n, t in kernel.params if isinstance(t, ir.TensorType)]
    if len(tensors) != 2 or len(kernel.params) != 2 or any(t.rank != 2 for _, t in tensors):
        return None
    dtype = tensors[0][1].dtype
    if dtype not in (F16, BF16, F32) or tensors[1][1].dtype != dtype:
        return None
    try:
        flow = df.evaluate(kernel)
    except (df.Unsupported, KeyError, IndexError, TypeError):
        return None
    if len(flow.stores) != 1:
        return None
    y, y_slices, stored = flow.stores[0]
    if len(y_slices) != 2:
        return None
    rows, cols = y_slices
    r = rows[1]
    if rows[2] or rows[0] != ("bin", "*", *sorted((("block", "x"), ("const", float(r))), key=repr)):
        return None
    if dtype != F32:
        if stored[0] != "cast" or stored[1] != dtype:
            return None
        stored = stored[2]

    def value(load: tuple) -> tuple | None:
        """v for a load of x at these slices: widened to f32 (f16/bf16) or read as it is (f32)."""
        inner = load[2] if dtype != F32 and load[0] == "cast" and load[1] == F32 else load
        if dtype != F32 and inner is load:
            return None
        return inner if inner[0] == "load" else None

    if not (stored[0] == "bin" and stored[1] == "/"):
        return None
    numerator, denominator = stored[2], stored[3]
    if not (numerator[0] == "math" and numerator[1] == "exp" and numerator[2][0] == "bin" and numerator[2][1] == "-"):
        return None
    v, shift = numerator[2][2], numerator[2][3]
    load = value(v)
    if load is None or load[2] != (rows, cols) or load[1] == y:
        return None
    x = load[1]
    if not flow.loops:
        # one tile: e = exp(v - rowmax(v)), y = e / rowsum(e)
        if cols[0] != ("const", 0.0) or cols[2] or shift != ("reduce", "max", 1, True, v):
            return None
        if denominator != ("reduce", "sum", 1, True, numerator):
            return None
        return SoftmaxPlan(x, y, dtype, int(r), int(cols[1]), False)
    if len(flow.loops) != 2:
        return None
    stats, out = flow.loops
    width = ("dim", x, 1)
    if not (_const(stats.lo, 0.0) and _const(out.lo, 0.0) and stats.hi == width and out.hi == width and
            stats.step == out.step == cols[1] and cols[0] == ("loopvar", out.var) and not out.init):
        return None
    if set(stats.init) != {shift[1], denominator[1]} or shift[0] != "final" or denominator[0] != "final":
        return None
    m, s = shift[1], denominator[1]
    if not (_fill_at_most(stats.init[m], -3.0e38) and stats.init[s] == ("fill", 0.0, (r, 1))):
        return None
    chunk = _substitute_loopvar(v, out.var, stats.var)
    m_new = ("math", "maximum", *sorted((("state", m), ("reduce", "max", 1, True, chunk)), key=repr))
    if stats.update[m] != m_new:
        return None
    rescaled = ("bin", "*", *sorted((("state", s), ("math", "exp", ("bin", "-", ("state", m), m_new))), key=repr))
    fresh = ("reduce", "sum", 1, True, ("math", "exp", ("bin", "-", chunk, m_new)))
    if stats.update[s] != ("bin", "+", *sorted((rescaled, fresh), key=repr)):
        return None
    return SoftmaxPlan(x, y, dtype, int(r), int(cols[1]), True)


def _fill_at_most(x: tuple, bound: float) -> bool:
    return x[0] in ("const", "fill") and not isinstance(x[1], bool) and x[1] <= bound


def _substitute_loopvar(value, old: str, new: str):
    """`value` with the loop variable `old` renamed `new` (the same chunk read by another loop)."""
    if value == ("loopvar", old):
        return ("loopvar", new)
    if isinstance(value, tuple):
        return tuple(_substitute_loopvar(x, old, new) for x in value)
    return value


def lower(kernel: ir.Kernel) -> GemmPlan | AttentionPlan | SoftmaxPlan | GenericPlan:
    """The plan for `kernel` on gfx950: a hand-written kernel when the program is one they serve, otherwise the
    generic HIP lowering."""
    return match_gemm(kernel) or match_attention(kernel) or match_softmax(kernel) or GenericPlan(kernel)


def why_generic(kernel: ir.Kernel) -> list[str]:
    """Why no hand-written kernel serves `kernel`: one line per specialised plan it did not match."""
    reasons = []
    if match_gemm(kernel) is None:
        reasons.append("not the whole-product GEMM: `acc = zeros`, one K loop `acc += a[rows, ks] @ b[cols, ks]"
                       ".transpose()` (or `b[ks, cols]`) of bf16/f16/fp8/int8 operands, one store of an epilogue of "
                       "scalar or row/column vector mul/add and relu/gelu/silu")
    if match_attention(kernel) is None:
        reasons.append("not krn's flash-attention program (its dataflow: an online softmax over key tiles with "
                       "exp2 or exp, an optional causal mask, head dimension 64 or 128, f16/bf16 tensors)")
    if match_softmax(kernel) is None:
        reasons.append("not krn's row softmax (its dataflow: exp(v - rowmax) / rowsum over one tile, or the running "
                       "maximum and sum over column chunks; f16, bf16 or f32)")
    return reasons

"""The oracle's C backend: tile IR -> C text -> clang -> ctypes, one C call per launch.

TEST INFRASTRUCTURE ONLY (see oracle/numerics.py). Also the CPU baseline that bench.py times.

Restates krn's CPU clang backend for the tile path (reference src/krn/runtime/cpu.py:92-152 and the lowering of
src/krn/compiler/emit.py): one C function runs the block grid as a loop nest, one thread per block (tile kernels
take bdim = 1, compiler/heuristics.py:175-176); every tile is a buffer; a matrix product stages both operands into
float32 buffers with invalid lanes as zero (emit.py:957-974) and then runs, for each output element,
`_s = fmaf(a[i*k+_k], b[_k*n+j], _s)` over `_k` in order (emit.py:788-796); a reduction walks its axis over the
valid lanes from the first one (emit.py:997-1034); stores are guarded. Flags follow cpu.py:48-51 and
compile_options.py:279-295: `-O2 -march=native -ffp-contract=off -fwrapv`.

This module writes its own C; the emitted text is not the reference's, its arithmetic is.
"""

import ctypes
import hashlib
import math
import os
import subprocess
import tempfile
import threading
from collections.abc import Sequence
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np

from krn_amd.compiler import ir
from krn_amd.compiler.space import geometry, runtime_args
from krn_amd.dtypes import BF16, BOOL, F16, F32, F64, I8, I32, I64, NUMPY, PY_FLOAT, PY_INT, Dtype, Kind
from krn_amd.frontend import Blocks

CLANG = next((c for c in ("/opt/rocm/lib/llvm/bin/clang", "clang", "gcc") if Path(c).exists() or c == "gcc"), "gcc")
FLAGS = ["-O2", "-march=native", "-ffp-contract=off", "-fwrapv", "-shared", "-fPIC", "-x", "c", "-lm"]
CACHE = Path(os.environ.get("KRN_ORACLE_CACHE", Path(tempfile.gettempdir()) / "krn_oracle_c"))


def ctype(dtype: Dtype) -> str:
    """C type of a tile element or scalar (bf16 held as a float value, fp8 as its code)."""
    if dtype.is_narrow:
        return "unsigned char"
    named = {
        BOOL: "unsigned char", F16: "_Float16", BF16: "float", F32: "float", F64: "double", PY_INT: "long long",
        PY_FLOAT: "double", I8: "signed char", I32: "int", I64: "long long",
    }  # fmt: skip
    if dtype in named:
        return named[dtype]
    if dtype.kind is Kind.UINT:
        return {8: "unsigned char", 16: "unsigned short", 32: "unsigned", 64: "unsigned long long"}[dtype.bits]
    return {8: "signed char", 16: "short", 32: "int", 64: "long long"}[dtype.bits]


def storage(dtype: Dtype) -> str:
    """C type of a tensor element in memory."""
    if dtype == BF16:
        return "unsigned short"
    return ctype(dtype)


PRELUDE = r"""
#include <math.h>
#include <stdlib.h>
#include <string.h>
static inline float kb16(float x) {  /* float32 -> nearest bf16 value, ties to even, NaN made quiet */
  unsigned u; memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) u = (u | 0x400000u) & 0xffff0000u;
  else u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  float y; memcpy(&y, &u, 4); return y;
}
static inline float kb16_load(unsigned short w) { unsigned u = (unsigned)w << 16; float y; memcpy(&y, &u, 4); return y; }
static inline unsigned short kb16_word(float x) { float y = kb16(x); unsigned u; memcpy(&u, &y, 4); return (unsigned short)(u >> 16); }
static inline float k8dec(unsigned char c) {  /* e4m3fn code -> value */
  int m = c & 7, e = (c >> 3) & 15; float v;
  if ((c & 0x7f) == 0x7f) return NAN;
  v = e ? ldexpf(1.0f + m / 8.0f, e - 7) : ldexpf(m / 8.0f, -6);
  return (c & 0x80) ? -v : v;
}
static inline unsigned char k8enc(float x) {  /* nearest e4m3fn code, ties to even, saturating, NaN -> 0x7f */
  if (x != x) return 0x7f;
  unsigned char sign = signbit(x) ? 0x80 : 0; float a = fabsf(x); if (a > 448.0f) a = 448.0f;
  int best = 0; float bd = INFINITY;
  for (int c = 0; c < 0x7f; ++c) { float d = fabsf(k8dec((unsigned char)c) - a);
    if (d < bd || (d == bd && (c % 2) == 0)) { bd = d; best = c; } }
  return sign | (unsigned char)best;
}
static inline float kmax(float a, float b) { return a != a ? a : b != b ? b : a > b ? a : b; }
static inline float kmin(float a, float b) { return a != a ? a : b != b ? b : a < b ? a : b; }
static inline float krelu(float x) { return x < 0.0f ? 0.0f : x; }
static inline float kgelu(float x) { return 0.5f * x * (1.0f + erff(x * 0.7071067811865476f)); }
static inline float ksilu(float x) { return x / (1.0f + expf(-x)); }
"""

MATH = {
    ir.Fn.EXP: "expf({0})", ir.Fn.EXP2: "exp2f({0})", ir.Fn.LOG: "logf({0})", ir.Fn.LOG2: "log2f({0})",
    ir.Fn.SQRT: "sqrtf({0})", ir.Fn.RSQRT: "(1.0f / sqrtf({0}))", ir.Fn.ABS: "fabsf({0})", ir.Fn.TANH: "tanhf({0})",
    ir.Fn.RELU: "krelu({0})", ir.Fn.GELU: "kgelu({0})", ir.Fn.SILU: "ksilu({0})",
    ir.Fn.SIGMOID: "(1.0f / (1.0f + expf(-({0}))))", ir.Fn.ERF: "erff({0})",
    ir.Fn.MAXIMUM: "kmax({0}, {1})", ir.Fn.MINIMUM: "kmin({0}, {1})",
}  # fmt: skip


class Emitter:
    def __init__(self, kernel: ir.Kernel) -> None:
        self.kernel = kernel
        self.lines: list[str] = []
        self.buffers: list[tuple[str, str, int]] = []  # (name, c type, count)
        self.depth = 2
        self.count = 0
        self.tile_vars: dict[str, tuple[str, str]] = {}

    def put(self, text: str) -> None:
        self.lines.append("    " * self.depth + text)

    def buffer(self, dtype: Dtype, shape: tuple[int, ...], stem: str = "t") -> tuple[str, str]:
        self.count += 1
        size = math.prod(shape) if shape else 1
        value, valid = f"{stem}{self.count}", f"{stem}{self.count}_v"
        self.buffers.append((value, ctype(dtype), size))
        self.buffers.append((valid, "unsigned char", size))
        return value, valid

    def loop(self, shape: tuple[int, ...], body) -> None:
        size = math.prod(shape)
        self.put(f"for (long long _e = 0; _e < {size}; ++_e) {{")
        self.depth += 1
        names = []
        for a in range(len(shape)):
            self.put(f"long long _i{a} = _e / {math.prod(shape[a + 1:])} % {shape[a]};")
            names.append(f"_i{a}")
        body(names)
        self.depth -= 1
        self.put("}")

    @staticmethod
    def index(shape: tuple[int, ...], idx: list[str], of: tuple[int, ...]) -> str:
        """Linear index into a tile of shape `of` broadcast to `shape`, numpy-style: aligned from the right."""
        if not of:
            return "0"
        skip = len(shape) - len(of)
        terms = []
        for a, extent in enumerate(of):
            if extent != 1:
                terms.append(f"{idx[a + skip]} * {math.prod(of[a + 1:])}")
        return " + ".join(terms) or "0"

    # ---- program

    def emit(self) -> str:
        for name, _ in self.kernel.params:
            pass
        for var in self.kernel.tiles:
            self.tile_vars[var.name] = self.buffer(var.dtype, var.shape, stem=f"v_{var.name.strip('_')}_")
        self.body(self.kernel.body)
        params = []
        for name, kind in self.kernel.params:
            for slot, dtype, role in ir.slots(name, kind):
                if role == "ptr":
                    params.append(f"{storage(dtype)}* restrict {slot}")
                else:
                    params.append(f"{ctype(dtype if dtype != I64 else PY_INT)} {slot}")
        params += ["long long gx", "long long gy", "long long gz", "long long first", "long long last"]
        total = sum(self.size(c) * n for _, c, n in self.buffers)
        head = [PRELUDE, f"void krn_{self.kernel.name}({', '.join(params)}) {{"]
        head.append(f"    char* _arena = (char*)aligned_alloc(64, {max(64, (total + len(self.buffers) * 64 + 63) // 64 * 64)});")
        offset = 0
        for name, c, n in self.buffers:
            head.append(f"    {c}* restrict {name} = ({c}*)(_arena + {offset});")
            offset += (self.size(c) * n + 63) // 64 * 64
        head.append("    for (long long _lin = first; _lin < last; ++_lin) {")
        head.append("        long long bx = _lin % gx, by = _lin / gx % gy, bz = _lin / (gx * gy);")
        head.append("        (void)bx; (void)by; (void)bz;")
        return "\n".join([*head, *self.lines, "    }", "    free(_arena);", "}", ""])

    @staticmethod
    def size(c: str) -> int:
        return {"unsigned char": 1, "signed char": 1, "_Float16": 2, "short": 2, "unsigned short": 2, "float": 4,
                "int": 4, "unsigned": 4, "double": 8, "long long": 8, "unsigned long long": 8}[c]

    def body(self, statements) -> None:
        for s in statements:
            getattr(self, f"stmt_{type(s).__name__}")(s)

    def stmt_TileAssign(self, s: ir.TileAssign) -> None:
        value, valid = self.tile(s.value)
        target, target_v = self.tile_vars[s.var.name]
        shape = s.var.shape

        def copy(idx):
            at = self.index(shape, idx, s.value.shape)
            self.put(f"{target}[_e] = {value}[{at}]; {target_v}[_e] = {valid}[{at}];")

        self.loop(shape, copy)

    def stmt_TileStore(self, s: ir.TileStore) -> None:
        value, valid = self.tile(s.value)
        tensor = s.tensor.name
        starts = [self.scalar(sl.start) for sl in s.slices]
        shape = s.value.shape
        self.put("{")
        self.depth += 1
        for a, start in enumerate(starts):
            self.put(f"long long _s{a} = {start};")

        def store(idx):
            tile_axes = iter(idx)
            cells = []
            for a, sl in enumerate(s.slices):
                cells.append(f"_s{a}" if sl.squeeze else f"(_s{a} + {next(tile_axes)})")
            inside = " && ".join(f"{c} >= 0 && {c} < {tensor}_n{a}" for a, c in enumerate(cells))
            linear = " + ".join(
                f"{c}" + "".join(f" * {tensor}_n{b}" for b in range(a + 1, len(cells))) for a, c in enumerate(cells))
            element = f"{value}[_e]"
            self.put(f"if ({valid}[_e] && {inside}) {tensor}[{linear}] = "
                     f"{self.to_storage(element, s.value.dtype, s.tensor.type.dtype)};")

        self.loop(shape, store)
        self.depth -= 1
        self.put("}")

    def to_storage(self, text: str, src: Dtype, dst: Dtype) -> str:
        if dst == BF16:
            return f"kb16_word({text})"
        return text

    def stmt_Accumulate(self, s: ir.Accumulate) -> None:
        acc, acc_v = self.tile_vars[s.acc.name]
        (m, k), n = s.lhs.shape, s.rhs.shape[1]
        integer = s.acc.dtype == I32
        stage = "int" if integer else "float"
        a, av = self.tile(s.lhs)
        b, bv = self.tile(s.rhs)
        af, bf = self.staged(stage, a, av, s.lhs), self.staged(stage, b, bv, s.rhs)
        self.put(f"for (long long _i = 0; _i < {m}; ++_i) for (long long _j = 0; _j < {n}; ++_j) {{")
        self.depth += 1
        if integer:
            self.put(f"unsigned _s = (unsigned){acc}[_i * {n} + _j];")
            self.put(f"for (long long _k = 0; _k < {k}; ++_k) _s += (unsigned)({af}[_i * {k} + _k] * {bf}[_k * {n} + _j]);")
            self.put(f"{acc}[_i * {n} + _j] = (int)_s;")
        else:
            self.put(f"float _s = {acc}[_i * {n} + _j];")
            self.put(f"for (long long _k = 0; _k < {k}; ++_k) _s = fmaf({af}[_i * {k} + _k], {bf}[_k * {n} + _j], _s);")
            self.put(f"{acc}[_i * {n} + _j] = _s;")
        self.depth -= 1
        self.put("}")
        # a row of the result with no valid lhs lane, or a column with no valid rhs lane, stays invalid
        self.put(f"for (long long _i = 0; _i < {m}; ++_i) {{ unsigned char _any = 0;"
                 f" for (long long _k = 0; _k < {k}; ++_k) _any |= {av}[_i * {k} + _k];"
                 f" if (!_any) for (long long _j = 0; _j < {n}; ++_j) {acc_v}[_i * {n} + _j] = 0; }}")
        self.put(f"for (long long _j = 0; _j < {n}; ++_j) {{ unsigned char _any = 0;"
                 f" for (long long _k = 0; _k < {k}; ++_k) _any |= {bv}[_k * {n} + _j];"
                 f" if (!_any) for (long long _i = 0; _i < {m}; ++_i) {acc_v}[_i * {n} + _j] = 0; }}")

    def staged(self, stage: str, value: str, valid: str, e: ir.Expr) -> str:
        """A float32 (int32 for int8) copy of a product operand with invalid lanes as zero."""
        self.count += 1
        name = f"st{self.count}"
        self.buffers.append((name, stage, math.prod(e.shape)))
        element = f"k8dec({value}[_e])" if e.dtype.is_narrow else f"({stage}){value}[_e]"
        self.put(f"for (long long _e = 0; _e < {math.prod(e.shape)}; ++_e) {name}[_e] = {valid}[_e] ? {element} : 0;")
        return name

    def stmt_For(self, s: ir.For) -> None:
        var = s.var.name
        self.put(f"for (long long {var} = {self.scalar(s.lo)}; {var} < {self.scalar(s.hi)}; {var} += {s.step}) {{")
        self.depth += 1
        self.body(s.body)
        self.depth -= 1
        self.put("}")

    def stmt_If(self, s: ir.If) -> None:
        self.put(f"if ({self.scalar(s.cond)}) {{")
        self.depth += 1
        self.body(s.then)
        self.depth -= 1
        self.put("} else {")
        self.depth += 1
        self.body(s.orelse)
        self.depth -= 1
        self.put("}")

    def stmt_Assign(self, s: ir.Assign) -> None:
        self.put(f"{ctype(s.var.dtype)} {s.var.name} = {self.scalar(s.value)};")

    # ---- scalars

    def scalar(self, e: ir.Expr) -> str:
        match e:
            case ir.Const(value=v):
                if e.dtype == BOOL:
                    return "1" if v else "0"
                if e.dtype.is_float or e.dtype == PY_FLOAT:
                    return f"(({ctype(e.dtype)}){float(v)!r})"
                return f"(({ctype(e.dtype)}){int(v)}LL)"
            case ir.Var(name=n):
                return n
            case ir.Param(name=n):
                return n
            case ir.Dim(tensor=t, axis=a):
                return f"{t.name}_n{a}"
            case ir.BlockIndex(axis=a):
                return f"b{a}"
            case ir.Cast(operand=o):
                return self.cast(self.scalar(o), o.dtype, e.dtype)
            case ir.Unary(op=ir.Op.NEG, operand=o):
                return f"(-{self.scalar(o)})"
            case ir.Binary(op=op, lhs=a, rhs=b):
                return f"({self.scalar(a)} {op.value if op not in (ir.Op.AND, ir.Op.OR) else op.value * 2} " \
                       f"{self.scalar(b)})"
        raise NotImplementedError(f"scalar {type(e).__name__}")

    def cast(self, text: str, src: Dtype, dst: Dtype) -> str:
        if src == dst:
            return text
        if src.is_narrow:
            text, src = f"k8dec({text})", F32
        if dst.is_narrow:
            return f"k8enc((float)({text}))"
        if dst == BF16:
            return f"kb16((float)({text}))"
        if dst == BOOL:
            return f"(({text}) != 0)"
        return f"(({ctype(dst)})({text}))"

    # ---- tiles: every expression materializes into a value buffer and a validity buffer

    def tile(self, e: ir.Expr) -> tuple[str, str]:
        if isinstance(e, ir.Var):
            return self.tile_vars[e.name]
        if not e.shape:
            value, valid = self.buffer(e.dtype, ())
            self.put(f"{value}[0] = {self.scalar(e)}; {valid}[0] = 1;")
            return value, valid
        return getattr(self, f"tile_{type(e).__name__}")(e)

    def tile_Zeros(self, e: ir.Zeros):
        value, valid = self.buffer(e.dtype, e.shape)
        self.loop(e.shape, lambda idx: self.put(f"{value}[_e] = 0; {valid}[_e] = 1;"))
        return value, valid

    def tile_TileLoad(self, e: ir.TileLoad):
        value, valid = self.buffer(e.dtype, e.shape)
        tensor = e.tensor.name
        self.put("{")
        self.depth += 1
        for a, sl in enumerate(e.slices):
            self.put(f"long long _s{a} = {self.scalar(sl.start)};")

        def load(idx):
            tile_axes = iter(idx)
            cells = [f"_s{a}" if sl.squeeze else f"(_s{a} + {next(tile_axes)})" for a, sl in enumerate(e.slices)]
            inside = " && ".join(f"{c} >= 0 && {c} < {tensor}_n{a}" for a, c in enumerate(cells))
            linear = " + ".join(
                f"{c}" + "".join(f" * {tensor}_n{b}" for b in range(a + 1, len(cells))) for a, c in enumerate(cells))
            element = f"{tensor}[{linear}]"
            if e.dtype == BF16:
                element = f"kb16_load({element})"
            self.put(f"if ({inside}) {{ {value}[_e] = {element}; {valid}[_e] = 1; }} "
                     f"else {{ {value}[_e] = 0; {valid}[_e] = 0; }}")

        self.loop(e.shape, load)
        self.depth -= 1
        self.put("}")
        return value, valid

    def tile_Transpose(self, e: ir.Transpose):
        a, av = self.tile(e.operand)
        value, valid = self.buffer(e.dtype, e.shape)
        rows, cols = e.operand.shape

        def copy(idx):
            src = f"{idx[1]} * {cols} + {idx[0]}"
            self.put(f"{value}[_e] = {a}[{src}]; {valid}[_e] = {av}[{src}];")

        self.loop(e.shape, copy)
        return value, valid

    def tile_Arange(self, e: ir.Arange):
        value, valid = self.buffer(e.dtype, e.shape)
        start = self.scalar(e.start)
        self.loop(e.shape, lambda idx: self.put(f"{value}[_e] = (int)({start} + {idx[e.axis]}); {valid}[_e] = 1;"))
        return value, valid

    def elementwise(self, e: ir.Expr, operands: list[ir.Expr], make) -> tuple[str, str]:
        parts = [self.tile(o) for o in operands]
        value, valid = self.buffer(e.dtype, e.shape)

        def body(idx):
            texts, checks = [], []
            for (v, vv), o in zip(parts, operands):
                at = self.index(e.shape, idx, o.shape)
                texts.append(f"{v}[{at}]")
                checks.append(f"{vv}[{at}]")
            self.put(f"{value}[_e] = {make(texts)}; {valid}[_e] = {' & '.join(checks)};")

        self.loop(e.shape, body)
        return value, valid

    def rounded(self, text: str, dtype: Dtype) -> str:
        return f"kb16({text})" if dtype == BF16 else f"({ctype(dtype)})({text})"

    def tile_Cast(self, e: ir.Cast):
        return self.elementwise(e, [e.operand], lambda t: self.cast(t[0], e.operand.dtype, e.dtype))

    def tile_Unary(self, e: ir.Unary):
        return self.elementwise(e, [e.operand], lambda t: self.rounded(f"-{t[0]}", e.dtype))

    def tile_Binary(self, e: ir.Binary):
        op = {ir.Op.AND: "&", ir.Op.OR: "|"}.get(e.op, e.op.value)
        if e.op is ir.Op.MOD and e.lhs.dtype.is_float:
            return self.elementwise(e, [e.lhs, e.rhs], lambda t: f"fmodf({t[0]}, {t[1]})")
        if e.op in ir.COMPARISONS:
            return self.elementwise(e, [e.lhs, e.rhs], lambda t: f"({t[0]} {op} {t[1]})")
        if e.op is ir.Op.DIV and e.lhs.dtype.is_int:
            return self.elementwise(e, [e.lhs, e.rhs], lambda t: f"({t[1]} ? {t[0]} / {t[1]} : 0)")
        return self.elementwise(e, [e.lhs, e.rhs], lambda t: self.rounded(f"{t[0]} {op} {t[1]}", e.dtype))

    def tile_Math(self, e: ir.Math):
        template = MATH[e.fn]
        if e.dtype == F64:
            template = template.replace("f(", "(")
        return self.elementwise(e, list(e.args), lambda t: self.rounded(template.format(*t), e.dtype))

    def tile_Select(self, e: ir.Select):
        return self.elementwise(e, [e.cond, e.then, e.orelse], lambda t: f"({t[0]} ? {t[1]} : {t[2]})")

    def tile_Reduce(self, e: ir.Reduce):
        a, av = self.tile(e.operand)
        value, valid = self.buffer(e.dtype, e.shape)
        shape, axis = e.operand.shape, e.axis
        count = shape[axis]
        reducer = {
            ir.Reduction.MAX: "_acc = (_x > _acc || _x != _x) ? _x : _acc;",
            ir.Reduction.MIN: "_acc = (_x < _acc || _x != _x) ? _x : _acc;",
            ir.Reduction.SUM: "_acc = _acc + _x;",
        }[e.op]
        if e.dtype == BF16:
            reducer = reducer.replace("_acc + _x", "kb16(_acc + _x)")

        def run(idx):
            full = list(idx) if e.keepdims else [*idx[:axis], "0", *idx[axis:]]
            full[axis] = "_r"
            at = self.index(shape, full, shape)
            self.put(f"{ctype(e.dtype)} _acc = 0; unsigned char _seen = 0;")
            self.put(f"for (long long _r = 0; _r < {count}; ++_r) {{ if (!{av}[{at}]) continue; "
                     f"{ctype(e.dtype)} _x = {a}[{at}]; if (_seen) {{ {reducer} }} else {{ _acc = _x; _seen = 1; }} }}")
            self.put(f"{value}[_e] = _acc; {valid}[_e] = _seen;")

        self.loop(e.shape, run)
        return value, valid


_lock = threading.Lock()


def compile_kernel(kernel: ir.Kernel) -> tuple[ctypes.CDLL, str]:
    """Compile the C text of `kernel` (cached by its digest) and return the library and the source."""
    source = Emitter(kernel).emit()
    digest = hashlib.sha256((source + " ".join(FLAGS) + CLANG).encode()).hexdigest()[:24]
    CACHE.mkdir(parents=True, exist_ok=True)
    library = CACHE / f"{kernel.name}_{digest}.so"
    with _lock:
        if not library.exists():
            c_file = CACHE / f"{kernel.name}_{digest}.c"
            c_file.write_text(source)
            temporary = library.with_suffix(f".{os.getpid()}.tmp")
            result = subprocess.run([CLANG, *FLAGS[:4], "-shared", "-fPIC", "-x", "c", str(c_file), "-o",
                                     str(temporary), "-lm"], capture_output=True, text=True)
            if result.returncode:
                raise RuntimeError(f"C backend compile failed:\n{result.stderr}\n{source}")
            temporary.replace(library)
    return ctypes.CDLL(str(library)), source


class Program:
    """A compiled kernel: call it with numpy arrays and scalars, like a krn CPU launch."""

    def __init__(self, kernel: ir.Kernel) -> None:
        self.kernel = kernel
        self.library, self.source = compile_kernel(kernel)
        self.function = getattr(self.library, f"krn_{kernel.name}")
        self.function.restype = None

    def arguments(self, args: Sequence[object]) -> list[object]:
        values = runtime_args(self.kernel, args)
        out: list[object] = []
        for (name, kind), value in zip(self.kernel.params, values):
            if isinstance(kind, ir.TensorType):
                array = value
                want = NUMPY[kind.dtype]
                if not isinstance(array, np.ndarray) or array.dtype != want or array.ndim != kind.rank:
                    raise TypeError(f"{self.kernel.name}: `{name}` needs a rank-{kind.rank} {want} array")
                if not array.flags.c_contiguous:
                    raise ValueError(f"`{name}` must be C-contiguous")
                out.append(ctypes.c_void_p(array.ctypes.data))
                out.extend(ctypes.c_longlong(d) for d in array.shape)
            elif kind.is_float:
                out.append(ctypes.c_double(value) if kind == F64 else ctypes.c_float(value))
            else:
                out.append(ctypes.c_longlong(int(value)) if kind.bits == 64 else ctypes.c_int(int(value)))
        return out

    def __call__(self, *args: object, launch: Blocks | None = None, threads: int = 1) -> None:
        values = runtime_args(self.kernel, args)
        grid = launch if launch is not None else geometry(self.kernel, values)
        native = self.arguments(args)
        blocks = grid.x * grid.y * grid.z
        dims = [ctypes.c_longlong(grid.x), ctypes.c_longlong(grid.y), ctypes.c_longlong(grid.z)]
        self.run_range(native, dims, 0, blocks, threads)

    def run_range(self, native, dims, first: int, last: int, threads: int = 1) -> None:
        """Blocks [first, last) of the grid; with threads > 1 the range is split across host threads (the C call
        releases the GIL), which is the N-core CPU baseline."""
        if threads <= 1 or last - first <= 1:
            self.function(*native, *dims, ctypes.c_longlong(first), ctypes.c_longlong(last))
            return
        bounds = np.linspace(first, last, min(threads, last - first) + 1).astype(int)
        with ThreadPoolExecutor(len(bounds) - 1) as pool:
            list(pool.map(lambda lo_hi: self.function(*native, *dims, ctypes.c_longlong(int(lo_hi[0])),
                                                      ctypes.c_longlong(int(lo_hi[1]))),
                          zip(bounds[:-1], bounds[1:])))


def run(kernel: ir.Kernel, launch: Blocks | None, args: Sequence[object], threads: int = 1) -> None:
    Program(kernel)(*args, launch=launch, threads=threads)

"""Generic lowering of any captured tile program to HIP C++ for gfx950, compiled at run time with hiprtc.

This is the path for tile programs that are not one of the contraction shapes the hand-written MFMA kernels serve
(`cdna4.lower` decides). One workgroup of 256 threads runs one block; every tile lives in LDS with a validity byte
per lane; each tile statement is an element loop strided over the workgroup followed by a barrier. Its arithmetic is
the tile semantics of krn's C-family lowering (reference src/krn/compiler/emit.py): a product stages both operands
as float32 (invalid lanes zero) and runs one fused multiply-add per k in k order for each output element
(emit.py:788-796), a reduction walks its axis over the valid lanes from the first one (emit.py:997-1034), stores
skip invalid lanes and elements outside the tensor. The kernel ABI is krn's generated-kernel ABI
(reference src/krn/compiler/cuda.py:319 and ir.py:441-452): `extern "C" __global__`, a tensor is a pointer plus one
`long long` extent per axis, scalars by value.
"""

import math
from dataclasses import dataclass

from krn_amd.compiler import ir
from krn_amd.dtypes import BF16, BOOL, F8E4M3, F16, F32, F64, I8, I32, I64, PY_FLOAT, PY_INT, Dtype, Kind

THREADS = 256
LDS_LIMIT = 160 * 1024


class LoweringError(ValueError):
    """A tile program the generic gfx950 lowering does not cover."""


def ctype(dtype: Dtype) -> str:
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
    return "unsigned short" if dtype == BF16 else ctype(dtype)


SIZES = {"unsigned char": 1, "signed char": 1, "_Float16": 2, "short": 2, "unsigned short": 2, "float": 4, "int": 4,
         "unsigned": 4, "double": 8, "long long": 8, "unsigned long long": 8}

PRELUDE = r"""
typedef unsigned int u32;
typedef _Float16 _k_half4 __attribute__((ext_vector_type(4)));
typedef short _k_short4 __attribute__((ext_vector_type(4)));
typedef _Float16 _k_half8 __attribute__((ext_vector_type(8)));
typedef __bf16 _k_bf16x8 __attribute__((ext_vector_type(8)));
typedef float _k_float4 __attribute__((ext_vector_type(4)));
typedef int _k_int4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float kb16(float x) {
  u32 u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) u = (u | 0x400000u) & 0xffff0000u;
  else u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  return __uint_as_float(u);
}
__device__ __forceinline__ float kb16_load(unsigned short w) { return __uint_as_float((u32)w << 16); }
__device__ __forceinline__ unsigned short kb16_word(float x) { return (unsigned short)(__float_as_uint(kb16(x)) >> 16); }
__device__ __forceinline__ float k8dec(unsigned char c) {
  int m = c & 7, e = (c >> 3) & 15;
  if ((c & 0x7f) == 0x7f) return __builtin_nanf("");
  float v = e ? ldexpf(1.0f + m * 0.125f, e - 7) : ldexpf(m * 0.125f, -6);
  return (c & 0x80) ? -v : v;
}
__device__ __forceinline__ unsigned char k8enc(float x) {
  if (x != x) return 0x7f;
  unsigned char sign = signbit(x) ? 0x80 : 0;
  float a = fabsf(x);
  if (a > 448.0f) a = 448.0f;
  int best = 0; float bd = __builtin_inff();
  for (int c = 0; c < 0x7f; ++c) {
    float d = fabsf(k8dec((unsigned char)c) - a);
    if (d < bd || (d == bd && (c & 1) == 0)) { bd = d; best = c; }
  }
  return sign | (unsigned char)best;
}
__device__ __forceinline__ float kmax(float a, float b) { return a != a ? a : b != b ? b : a > b ? a : b; }
__device__ __forceinline__ float kmin(float a, float b) { return a != a ? a : b != b ? b : a < b ? a : b; }
// activations as krn states them (reference compiler/emit.py:112-114)
__device__ __forceinline__ float krelu(float x) { return x < 0.0f ? 0.0f : x; }
__device__ __forceinline__ float kgelu(float x) { return 0.5f * x * (1.0f + erff(x * 0.7071067811865476f)); }
__device__ __forceinline__ float ksilu(float x) { return x / (1.0f + expf(-x)); }
"""

MATH = {
    ir.Fn.EXP: "expf({0})", ir.Fn.EXP2: "exp2f({0})", ir.Fn.LOG: "logf({0})", ir.Fn.LOG2: "log2f({0})",
    ir.Fn.SQRT: "sqrtf({0})", ir.Fn.RSQRT: "(1.0f / sqrtf({0}))", ir.Fn.ABS: "fabsf({0})", ir.Fn.TANH: "tanhf({0})",
    ir.Fn.RELU: "krelu({0})", ir.Fn.GELU: "kgelu({0})", ir.Fn.SILU: "ksilu({0})",
    ir.Fn.SIGMOID: "(1.0f / (1.0f + expf(-({0}))))", ir.Fn.ERF: "erff({0})",
    ir.Fn.MAXIMUM: "kmax({0}, {1})", ir.Fn.MINIMUM: "kmin({0}, {1})",
}  # fmt: skip


@dataclass(frozen=True)
class MfmaForm:
    """A 16 x 16 x K_STEP matrix-core instruction the generic lowering uses for a product."""

    name: str
    builtin: str
    k_step: int
    element: str  # the staged operand element
    operand_vec: str  # one lane's operand of one instruction
    acc_vec: str
    integer: bool = False


# per operand type, the forms in order of preference: gfx950's 16x16x32 f16/bf16 instructions consume twice the K of
# the 16x16x16 ones (kept for products whose K is a multiple of 16 only); fp8 e4m3 (the OCP format on gfx950) and
# int8 consume 32 bytes of K per instruction
MFMA_FORMS = {
    F16: (MfmaForm("f16", "__builtin_amdgcn_mfma_f32_16x16x32_f16", 32, "unsigned short", "_k_half8", "_k_float4"),
          MfmaForm("f16", "__builtin_amdgcn_mfma_f32_16x16x16f16", 16, "unsigned short", "_k_half4", "_k_float4")),
    BF16: (MfmaForm("bf16", "__builtin_amdgcn_mfma_f32_16x16x32_bf16", 32, "unsigned short", "_k_bf16x8",
                    "_k_float4"),
           MfmaForm("bf16", "__builtin_amdgcn_mfma_f32_16x16x16bf16_1k", 16, "unsigned short", "_k_short4",
                    "_k_float4")),
    F8E4M3: (MfmaForm("fp8", "__builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8", 32, "unsigned char", "long",
                      "_k_float4"),),
    I8: (MfmaForm("i8", "__builtin_amdgcn_mfma_i32_16x16x32_i8", 32, "signed char", "long", "_k_int4", True),),
}


def mfma_form(s: ir.Accumulate) -> MfmaForm | None:
    """The matrix-core instruction for a product, when its operand types have one and the tile extents are whole
    instructions (m and n multiples of 16, k of the instruction's K); None keeps the scalar fused multiply-adds.
    f16/bf16/fp8 products accumulate in float32, int8 ones in int32 (exact, so any order gives the same result)."""
    (m, k), n = s.lhs.shape, s.rhs.shape[1]
    if s.lhs.dtype != s.rhs.dtype or s.lhs.dtype not in MFMA_FORMS or m % 16 or n % 16:
        return None
    for form in MFMA_FORMS[s.lhs.dtype]:
        if (s.acc.dtype == I32) != form.integer or (not form.integer and s.acc.dtype != F32):
            continue
        if k % form.k_step == 0:
            return form
    return None


def products(kernel: ir.Kernel) -> list[str]:
    """How the generic lowering runs each product of `kernel`: "mfma 16x16x<K> <type>" or "scalar fma"."""
    found: list[str] = []

    def walk(statements) -> None:
        for s in statements:
            if isinstance(s, ir.Accumulate):
                form = mfma_form(s)
                found.append(f"mfma 16x16x{form.k_step} {form.name}" if form else "scalar fma")
            for field_name in ("body", "then", "orelse"):
                walk(getattr(s, field_name, ()) or ())

    walk(kernel.body)
    return found


class Emitter:
    def __init__(self, kernel: ir.Kernel, entry: str) -> None:
        self.kernel, self.entry = kernel, entry
        self.mfma_products = 0
        self.lines: list[str] = []
        self.buffers: list[tuple[str, str, int]] = []
        self.depth = 1
        self.count = 0
        self.tile_vars: dict[str, tuple[str, str]] = {}

    def put(self, text: str) -> None:
        self.lines.append("  " * self.depth + text)

    def buffer(self, dtype: Dtype, shape: tuple[int, ...], stem: str = "t") -> tuple[str, str]:
        self.count += 1
        size = math.prod(shape) if shape else 1
        value, valid = f"{stem}{self.count}", f"{stem}{self.count}_v"
        self.buffers.append((value, ctype(dtype), size))
        self.buffers.append((valid, "unsigned char", size))
        return value, valid

    def loop(self, shape: tuple[int, ...], body) -> None:
        size = math.prod(shape)
        self.put(f"for (int _e = threadIdx.x; _e < {size}; _e += {THREADS}) {{")
        self.depth += 1
        names = []
        for a in range(len(shape)):
            self.put(f"const int _i{a} = _e / {math.prod(shape[a + 1:])} % {shape[a]};")
            names.append(f"_i{a}")
        body(names)
        self.depth -= 1
        self.put("}")
        self.put("__syncthreads();")

    @staticmethod
    def index(idx: list[str], of: tuple[int, ...]) -> str:
        """Linear index into a tile of shape `of` broadcast numpy-style (aligned from the right) to the loop `idx`."""
        if not of:
            return "0"
        skip = len(idx) - len(of)
        terms = [f"{idx[a + skip]} * {math.prod(of[a + 1:])}" for a, extent in enumerate(of) if extent != 1]
        return " + ".join(terms) or "0"

    def emit(self) -> tuple[str, int]:
        for var in self.kernel.tiles:
            self.tile_vars[var.name] = self.buffer(var.dtype, var.shape, stem=f"v_{var.name.strip('_')}_")
        self.body(self.kernel.body)
        params = []
        for name, kind in self.kernel.params:
            for slot, dtype, role in ir.slots(name, kind):
                if role == "ptr":
                    params.append(f"{storage(dtype)}* __restrict__ {slot}")
                else:
                    params.append(f"{ctype(dtype if dtype != I64 else PY_INT)} {slot}")
        total = sum((SIZES[c] * n + 15) // 16 * 16 for _, c, n in self.buffers)
        scratch = total > LDS_LIMIT  # tiles beyond one CU's LDS live in a per-block slice of global scratch
        if scratch:
            params.append("char* __restrict__ _scratch")
        head = [PRELUDE, f'extern "C" __global__ __launch_bounds__({THREADS}) void {self.entry}({", ".join(params)}) {{']
        if scratch:
            head.append(f"  char* _block = _scratch + ((long long)blockIdx.x + (long long)blockIdx.y * gridDim.x + "
                        f"(long long)blockIdx.z * gridDim.x * gridDim.y) * {total}LL;")
            offset = 0
            for name, c, n in self.buffers:
                head.append(f"  {c}* __restrict__ {name} = ({c}*)(_block + {offset});")
                offset += (SIZES[c] * n + 15) // 16 * 16
        else:
            head += [f"  __shared__ __attribute__((aligned(16))) {c} {name}[{n}];" for name, c, n in self.buffers]
        self.scratch_bytes = total if scratch else 0
        head += ["  const long long bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;",
                 "  (void)bx; (void)by; (void)bz;"]
        return "\n".join([*head, *self.lines, "}", ""]), self.scratch_bytes

    def body(self, statements) -> None:
        for s in statements:
            getattr(self, f"stmt_{type(s).__name__}")(s)

    def stmt_TileAssign(self, s: ir.TileAssign) -> None:
        value, valid = self.tile(s.value)
        target, target_v = self.tile_vars[s.var.name]
        if (value, valid) == (target, target_v):
            return
        # a value that reads the variable it assigns is computed into a temporary first (one barrier between)
        self.loop(s.var.shape, lambda idx: self.put(
            f"{target}[_e] = {value}[{self.index(idx, s.value.shape)}]; "
            f"{target_v}[_e] = {valid}[{self.index(idx, s.value.shape)}];"))

    def stmt_TileStore(self, s: ir.TileStore) -> None:
        value, valid = self.tile(s.value)
        tensor = s.tensor.name
        starts = [f"_s{a}" for a in range(len(s.slices))]
        for a, sl in enumerate(s.slices):
            self.put(f"{{ const long long _s{a} = {self.scalar(sl.start)};")

        def store(idx):
            axes = iter(idx)
            cells = [st if sl.squeeze else f"({st} + {next(axes)})" for st, sl in zip(starts, s.slices)]
            inside = " && ".join(f"{c} >= 0 && {c} < {tensor}_n{a}" for a, c in enumerate(cells))
            linear = " + ".join(c + "".join(f" * {tensor}_n{b}" for b in range(a + 1, len(cells)))
                                for a, c in enumerate(cells))
            element = f"{value}[_e]"
            if s.tensor.type.dtype == BF16:
                element = f"kb16_word({element})"
            self.put(f"if ({valid}[_e] && {inside}) {tensor}[{linear}] = {element};")

        self.loop(s.value.shape, store)
        self.put("}" * len(s.slices))

    def stmt_Accumulate(self, s: ir.Accumulate) -> None:
        acc, acc_v = self.tile_vars[s.acc.name]
        (m, k), n = s.lhs.shape, s.rhs.shape[1]
        integer = s.acc.dtype == I32
        stage = "int" if integer else "float"
        a, av = self.tile(s.lhs)
        b, bv = self.tile(s.rhs)
        form = mfma_form(s)
        if form is not None:
            self.mfma_product(s, form, (a, av), (b, bv), (acc, acc_v))
            return
        af, bf = self.staged(stage, a, av, s.lhs), self.staged(stage, b, bv, s.rhs)
        self.put(f"for (int _e = threadIdx.x; _e < {m * n}; _e += {THREADS}) {{")
        self.put(f"  const int _i = _e / {n}, _j = _e % {n};")
        if integer:
            self.put(f"  unsigned _s = (unsigned){acc}[_e];")
            self.put(f"  for (int _k = 0; _k < {k}; ++_k) _s += (unsigned)({af}[_i * {k} + _k] * {bf}[_k * {n} + _j]);")
            self.put(f"  {acc}[_e] = (int)_s;")
        else:
            self.put(f"  float _s = {acc}[_e];")
            self.put(f"  for (int _k = 0; _k < {k}; ++_k) _s = fmaf({af}[_i * {k} + _k], {bf}[_k * {n} + _j], _s);")
            self.put(f"  {acc}[_e] = _s;")
        self.put(f"  unsigned char _row = 0, _col = 0;")
        self.put(f"  for (int _k = 0; _k < {k}; ++_k) {{ _row |= {av}[_i * {k} + _k]; _col |= {bv}[_k * {n} + _j]; }}")
        self.put(f"  {acc_v}[_e] = {acc_v}[_e] & _row & _col;")
        self.put("}")
        self.put("__syncthreads();")

    def mfma_product(self, s: ir.Accumulate, form: "MfmaForm", lhs, rhs, accumulator) -> None:
        """acc[m, n] += lhs[m, k] @ rhs[k, n] on the matrix cores: both operands staged into LDS K-contiguous as the
        instruction's operand type (invalid lanes 0, so they add nothing), then each of the 4 waves takes 16 x 16
        output blocks in turn, loads the block's accumulators, runs k / K_STEP MFMAs and writes them back. Lane l of
        a 16x16xK MFMA holds operand row (or column) l % 16 and K_STEP / 4 consecutive k from (l / 16) * K_STEP / 4,
        and accumulators rows 4 (l / 16) + i, column l % 16 (reference compiler/hip.py:70-97 `AMDMFMA.product`,
        compiler/emit.py:924-955 `matrix_stage`). The validity of the accumulator is the scalar path's."""
        (a, av), (b, bv), (acc, acc_v) = lhs, rhs, accumulator
        (m, k), n = s.lhs.shape, s.rhs.shape[1]
        per = form.k_step // 4  # operand elements per lane per instruction
        at = self.mfma_stage(form, a, av, s.lhs, m, k, transposed=False)
        bt = self.mfma_stage(form, b, bv, s.rhs, n, k, transposed=True)
        acc_t = "int" if form.integer else "float"
        self.put("{")
        self.put("  const int _w = threadIdx.x >> 6, _l = threadIdx.x & 63, _r = _l & 15, _q = _l >> 4;")
        self.put(f"  for (int _blk = _w; _blk < {(m // 16) * (n // 16)}; _blk += {THREADS // 64}) {{")
        self.put(f"    const int _m0 = (_blk / {n // 16}) * 16, _n0 = (_blk % {n // 16}) * 16;")
        self.put(f"    {form.acc_vec} _c;")
        self.put(f"    for (int _i = 0; _i < 4; ++_i) _c[_i] = {acc}[(_m0 + 4 * _q + _i) * {n} + _n0 + _r];")
        self.put(f"    for (int _k = 0; _k < {k}; _k += {form.k_step}) {{")
        self.put(f"      const {form.operand_vec} _a = *(const {form.operand_vec}*)&{at}[(_m0 + _r) * {k} + _k + _q * {per}];")
        self.put(f"      const {form.operand_vec} _b = *(const {form.operand_vec}*)&{bt}[(_n0 + _r) * {k} + _k + _q * {per}];")
        self.put(f"      _c = {form.builtin}(_a, _b, _c, 0, 0, 0);")
        self.put("    }")
        self.put(f"    for (int _i = 0; _i < 4; ++_i) {acc}[(_m0 + 4 * _q + _i) * {n} + _n0 + _r] = ({acc_t})_c[_i];")
        self.put("  }")
        self.put("}")
        self.put(f"for (int _e = threadIdx.x; _e < {m * n}; _e += {THREADS}) {{")
        self.put(f"  const int _i = _e / {n}, _j = _e % {n};")
        self.put(f"  unsigned char _row = 0, _col = 0;")
        self.put(f"  for (int _k = 0; _k < {k}; ++_k) {{ _row |= {av}[_i * {k} + _k]; _col |= {bv}[_k * {n} + _j]; }}")
        self.put(f"  {acc_v}[_e] = {acc_v}[_e] & _row & _col;")
        self.put("}")
        self.put("__syncthreads();")
        self.mfma_products += 1

    def mfma_stage(self, form: "MfmaForm", value: str, valid: str, e: ir.Expr, rows: int, k: int,
                   transposed: bool) -> str:
        """An operand in LDS as `rows` K-contiguous rows of the instruction's element bits; `transposed` reads a
        (k, rows) tile."""
        self.count += 1
        name = f"mf{self.count}"
        self.buffers.append((name, form.element, rows * k))
        source = f"{value}[_kk * {rows} + _rr]" if transposed else f"{value}[_rr * {k} + _kk]"
        check = f"{valid}[_kk * {rows} + _rr]" if transposed else f"{valid}[_rr * {k} + _kk]"
        bits = {"f16": f"__builtin_bit_cast(unsigned short, (_Float16){source})",
                "bf16": f"(unsigned short)(__float_as_uint({source}) >> 16)",
                "fp8": f"(unsigned char){source}",  # the e4m3 code as the tile holds it
                "i8": f"(signed char){source}"}[form.name]
        self.put(f"for (int _e = threadIdx.x; _e < {rows * k}; _e += {THREADS}) {{")
        self.put(f"  const int _rr = _e / {k}, _kk = _e % {k};")
        self.put(f"  {name}[_e] = {check} ? {bits} : ({form.element})0;")
        self.put("}")
        self.put("__syncthreads();")
        return name

    def staged(self, stage: str, value: str, valid: str, e: ir.Expr) -> str:
        self.count += 1
        name = f"st{self.count}"
        self.buffers.append((name, stage, math.prod(e.shape)))
        element = f"k8dec({value}[_e])" if e.dtype.is_narrow else f"({stage}){value}[_e]"
        self.put(f"for (int _e = threadIdx.x; _e < {math.prod(e.shape)}; _e += {THREADS}) "
                 f"{name}[_e] = {valid}[_e] ? {element} : ({stage})0;")
        self.put("__syncthreads();")
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
        self.put(f"const {ctype(s.var.dtype)} {s.var.name} = {self.scalar(s.value)};")

    def scalar(self, e: ir.Expr) -> str:
        match e:
            case ir.Const(value=v):
                if e.dtype == BOOL:
                    return "1" if v else "0"
                if e.dtype.is_float or e.dtype == PY_FLOAT:
                    return f"(({ctype(e.dtype)}){float(v)!r})"
                return f"(({ctype(e.dtype)}){int(v)}LL)"
            case ir.Var(name=n) | ir.Param(name=n):
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
                symbol = {ir.Op.AND: "&&", ir.Op.OR: "||"}.get(op, op.value)
                return f"({self.scalar(a)} {symbol} {self.scalar(b)})"
        raise LoweringError(f"scalar {type(e).__name__} is not lowered")

    def cast(self, text: str, src: Dtype, dst: Dtype) -> str:
        if src == dst:
            return text
        if src.is_narrow:
            text = f"k8dec({text})"
        if dst.is_narrow:
            return f"k8enc((float)({text}))"
        if dst == BF16:
            return f"kb16((float)({text}))"
        if dst == BOOL:
            return f"(({text}) != 0)"
        return f"(({ctype(dst)})({text}))"

    def tile(self, e: ir.Expr) -> tuple[str, str]:
        if isinstance(e, ir.Var):
            return self.tile_vars[e.name]
        if not e.shape:
            value, valid = self.buffer(e.dtype, ())
            self.put(f"if (threadIdx.x == 0) {{ {value}[0] = {self.scalar(e)}; {valid}[0] = 1; }}")
            self.put("__syncthreads();")
            return value, valid
        return getattr(self, f"tile_{type(e).__name__}")(e)

    def tile_Zeros(self, e: ir.Zeros):
        value, valid = self.buffer(e.dtype, e.shape)
        self.loop(e.shape, lambda idx: self.put(f"{value}[_e] = 0; {valid}[_e] = 1;"))
        return value, valid

    def tile_TileLoad(self, e: ir.TileLoad):
        value, valid = self.buffer(e.dtype, e.shape)
        tensor = e.tensor.name
        starts = [f"_s{a}" for a in range(len(e.slices))]
        for a, sl in enumerate(e.slices):
            self.put(f"{{ const long long _s{a} = {self.scalar(sl.start)};")

        def load(idx):
            axes = iter(idx)
            cells = [st if sl.squeeze else f"({st} + {next(axes)})" for st, sl in zip(starts, e.slices)]
            inside = " && ".join(f"{c} >= 0 && {c} < {tensor}_n{a}" for a, c in enumerate(cells))
            linear = " + ".join(c + "".join(f" * {tensor}_n{b}" for b in range(a + 1, len(cells)))
                                for a, c in enumerate(cells))
            element = f"{tensor}[{linear}]"
            if e.dtype == BF16:
                element = f"kb16_load({element})"
            self.put(f"if ({inside}) {{ {value}[_e] = {element}; {valid}[_e] = 1; }} "
                     f"else {{ {value}[_e] = 0; {valid}[_e] = 0; }}")

        self.loop(e.shape, load)
        self.put("}" * len(e.slices))
        return value, valid

    def tile_Transpose(self, e: ir.Transpose):
        a, av = self.tile(e.operand)
        value, valid = self.buffer(e.dtype, e.shape)
        cols = e.operand.shape[1]
        self.loop(e.shape, lambda idx: self.put(
            f"{value}[_e] = {a}[{idx[1]} * {cols} + {idx[0]}]; {valid}[_e] = {av}[{idx[1]} * {cols} + {idx[0]}];"))
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
            texts = [f"{v}[{self.index(idx, o.shape)}]" for (v, _), o in zip(parts, operands)]
            checks = [f"{vv}[{self.index(idx, o.shape)}]" for (_, vv), o in zip(parts, operands)]
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
            at = self.index(full, shape)
            self.put(f"{ctype(e.dtype)} _acc = 0; unsigned char _seen = 0;")
            self.put(f"for (int _r = 0; _r < {shape[axis]}; ++_r) {{ if (!{av}[{at}]) continue; "
                     f"{ctype(e.dtype)} _x = {a}[{at}]; if (_seen) {{ {reducer} }} else {{ _acc = _x; _seen = 1; }} }}")
            self.put(f"{value}[_e] = _acc; {valid}[_e] = _seen;")

        self.loop(e.shape, run)
        return value, valid


def emit(kernel: ir.Kernel, entry: str) -> tuple[str, int]:
    """HIP source of `kernel` with the entry point `entry`, and the global scratch bytes each block needs (0 when
    its tiles fit in LDS; otherwise the kernel takes a trailing `_scratch` pointer to blocks x that many bytes)."""
    return Emitter(kernel, entry).emit()

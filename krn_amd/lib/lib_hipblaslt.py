"""hipBLASLt behind `lib.matmul`: the first AMD candidate of the reference's order (src/krn/lib/lib.py:264, adapter
name "hipblaslt" at lib.py:516), bound with ctypes to `libhipblaslt.so`.

Row-major `out (m x n) = a (m x k) @ b (k x n)` is column-major `out^T = b^T @ a^T`: hipBLASLt's A is b viewed as an
n x k column-major matrix, its B is a viewed as k x m, and D is out viewed as n x m, all untransposed, so no copy is
made. The bias broadcasts along D's rows, which are out's columns. Plans (descriptors, layouts and the top heuristic
algorithm) are cached per thread by dtypes, shape, epilogue and bias presence; the workspace is allocated once per
stream and kept with the plan. Problems hipBLASLt documents no kernel for are refused before planning, and a
heuristic that finds no algorithm declines, so the call falls to `ours`. (The same structure as the reference's
cuBLASLt adapter, src/krn/lib/lib_cublaslt.py, over the ROCm library and its enums.)
"""

import ctypes
import threading
import weakref
from ctypes import POINTER, byref, c_float, c_int, c_int64, c_size_t, c_uint32, c_uint64, c_void_p

from krn_amd.dtypes import BF16, F16, F32, U8
from krn_amd.hw import Libraries, LibraryNotFound
from krn_amd.lib.lib import Candidate, Declined, Epilogue, Op, Operands, Origin, Problem
from krn_amd.runtime.api import Stream

# hipDataType (hip/library_types.h) and hipblasComputeType_t (hipblas-common.h)
DATA_TYPES = {F32: 0, F16: 2, BF16: 14}
COMPUTE_32F = 2
# (a, b, out) triples with a float32-accumulating hipBLASLt kernel
FORMATS = {(F16, F16, F16), (F16, F16, F32), (BF16, BF16, BF16), (BF16, BF16, F32), (F32, F32, F32)}
# hipblasLtEpilogue_t (hipblaslt.h)
EPILOGUES = {
    Epilogue.NONE: 1,  # HIPBLASLT_EPILOGUE_DEFAULT
    Epilogue.RELU: 2,
    Epilogue.BIAS: 4,
    Epilogue.BIAS_RELU: 6,
    Epilogue.GELU: 32,
    Epilogue.BIAS_GELU: 36,
    Epilogue.SILU: 65536,  # HIPBLASLT_EPILOGUE_SWISH_EXT: x * sigmoid(x)
}
DESC_EPILOGUE, DESC_BIAS_POINTER, DESC_BIAS_DATA_TYPE = 2, 3, 4  # hipblasLtMatmulDescAttributes_t
PREF_MAX_WORKSPACE_BYTES = 1
WORKSPACE_BYTES = 32 << 20
STATUS = {0: "SUCCESS", 1: "NOT_INITIALIZED", 2: "ALLOC_FAILED", 3: "INVALID_VALUE", 4: "MAPPING_ERROR",
          5: "EXECUTION_FAILED", 6: "INTERNAL_ERROR", 7: "NOT_SUPPORTED", 8: "ARCH_MISMATCH",
          9: "HANDLE_IS_NULLPTR", 10: "INVALID_ENUM", 11: "UNKNOWN"}  # fmt: skip
UNSUPPORTED = (3, 7)


class Algo(ctypes.Structure):
    _fields_ = [("data", ctypes.c_uint8 * 16), ("max_workspace_bytes", c_size_t)]


class HeuristicResult(ctypes.Structure):
    _fields_ = [("algo", Algo), ("workspace_size", c_size_t), ("state", c_int), ("waves_count", c_float),
                ("reserved", c_int * 4)]


class HipblasLtError(RuntimeError):
    def __init__(self, function: str, status: int) -> None:
        self.function, self.status = function, status
        super().__init__(f"{function} failed with HIPBLAS_STATUS_{STATUS.get(status, status)}")


class _Api:
    def __init__(self) -> None:
        lib = Libraries.load("hipblaslt").handle
        signatures = {
            "hipblasLtCreate": [POINTER(c_void_p)],
            "hipblasLtDestroy": [c_void_p],
            "hipblasLtMatmulDescCreate": [POINTER(c_void_p), c_int, c_int],
            "hipblasLtMatmulDescDestroy": [c_void_p],
            "hipblasLtMatmulDescSetAttribute": [c_void_p, c_int, c_void_p, c_size_t],
            "hipblasLtMatrixLayoutCreate": [POINTER(c_void_p), c_int, c_uint64, c_uint64, c_int64],
            "hipblasLtMatrixLayoutDestroy": [c_void_p],
            "hipblasLtMatmulPreferenceCreate": [POINTER(c_void_p)],
            "hipblasLtMatmulPreferenceDestroy": [c_void_p],
            "hipblasLtMatmulPreferenceSetAttribute": [c_void_p, c_int, c_void_p, c_size_t],
            "hipblasLtMatmulAlgoGetHeuristic": [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                                c_int, POINTER(HeuristicResult), POINTER(c_int)],
            "hipblasLtMatmul": [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                c_void_p, c_void_p, c_void_p, c_void_p, POINTER(Algo), c_void_p, c_size_t, c_void_p],
        }  # fmt: skip
        for name, argtypes in signatures.items():
            function = getattr(lib, name)
            function.argtypes, function.restype = argtypes, c_int
        self.lib = lib

    def __call__(self, name: str, *args) -> None:
        status = getattr(self.lib, name)(*args)
        if status:
            raise HipblasLtError(name, status)

    def raw(self, name: str, *args) -> int:
        return getattr(self.lib, name)(*args)


_api: _Api | None = None


def api() -> _Api:
    global _api
    if _api is None:
        _api = _Api()
    return _api


def refusal(problem: Problem) -> str | None:
    names = ", ".join(str(d) for d in problem.dtypes)
    if problem.dtypes not in FORMATS:
        return f"hipBLASLt has float32-accumulating kernels for (f16|bf16, same, same|f32) and f32; got ({names})"
    if problem.epilogue not in EPILOGUES:
        return f"{problem.epilogue} has no hipBLASLt epilogue"
    if min(problem.shape) == 0:
        return "an empty product launches nothing"
    return None


class Plan:
    """Descriptors, layouts and the heuristic's algorithm for one problem; the workspace of each stream it ran on."""

    def __init__(self, handle: int, problem: Problem) -> None:
        m, n, k = problem.shape
        a_type, b_type, out_type = (DATA_TYPES[d] for d in problem.dtypes)
        lt = api()
        self._owned: list[tuple[str, int]] = []
        finalizer = weakref.finalize(self, _destroy, self._owned)
        try:
            desc = c_void_p()
            lt("hipblasLtMatmulDescCreate", byref(desc), COMPUTE_32F, DATA_TYPES[F32])
            self._owned.append(("hipblasLtMatmulDescDestroy", desc.value))
            self.desc = desc
            self._set(DESC_EPILOGUE, c_uint32(EPILOGUES[problem.epilogue]))
            if problem.epilogue.has_bias:
                self._set(DESC_BIAS_DATA_TYPE, c_int(out_type))
            self.bias = None
            self.layouts = []
            for dtype, rows, cols in ((b_type, n, k), (a_type, k, m), (out_type, n, m)):
                layout = c_void_p()
                lt("hipblasLtMatrixLayoutCreate", byref(layout), dtype, rows, cols, rows)
                self._owned.append(("hipblasLtMatrixLayoutDestroy", layout.value))
                self.layouts.append(layout)
            preference = c_void_p()
            lt("hipblasLtMatmulPreferenceCreate", byref(preference))
            self._owned.append(("hipblasLtMatmulPreferenceDestroy", preference.value))
            limit = c_uint64(WORKSPACE_BYTES)
            lt("hipblasLtMatmulPreferenceSetAttribute", preference, PREF_MAX_WORKSPACE_BYTES, byref(limit),
               ctypes.sizeof(limit))
            self.result, found = HeuristicResult(), c_int(0)
            left, right, out = self.layouts
            lt("hipblasLtMatmulAlgoGetHeuristic", c_void_p(handle), desc, left, right, out, out, preference, 1,
               byref(self.result), byref(found))
        except HipblasLtError as error:
            finalizer()
            if error.status in UNSUPPORTED:
                raise Declined(f"hipBLASLt has no algorithm for {problem}: {error}") from error
            raise
        if found.value == 0 or self.result.state != 0:
            finalizer()
            raise Declined(f"hipBLASLt's heuristic found no algorithm for {problem}")
        self.alpha, self.beta = c_float(1.0), c_float(0.0)
        self.workspaces: dict[int, object] = {}

    def _set(self, attribute: int, value) -> None:
        api()("hipblasLtMatmulDescSetAttribute", self.desc, attribute, byref(value), ctypes.sizeof(value))

    def workspace(self, stream) -> tuple[int, int]:
        size = self.result.workspace_size
        if size == 0:
            return 0, 0
        buffer = self.workspaces.get(stream.handle)
        if buffer is None:
            buffer = self.workspaces[stream.handle] = stream.device.empty_on(stream, U8, size)
        return buffer.pointer, size

    def enqueue(self, handle: int, operands: Operands, stream) -> None:
        if operands.bias is not None and operands.bias.pointer != self.bias:
            self._set(DESC_BIAS_POINTER, c_void_p(operands.bias.pointer))
            self.bias = operands.bias.pointer
        workspace, size = self.workspace(stream)
        left, right, out = self.layouts
        api()("hipblasLtMatmul", c_void_p(handle), self.desc, byref(self.alpha), c_void_p(operands.b.pointer), left,
              c_void_p(operands.a.pointer), right, byref(self.beta), c_void_p(operands.out.pointer), out,
              c_void_p(operands.out.pointer), out, byref(self.result.algo), c_void_p(workspace), size,
              c_void_p(stream.handle))


def _destroy(owned: list[tuple[str, int]]) -> None:
    for function, handle in reversed(owned):
        try:
            api().raw(function, c_void_p(handle))
        except Exception:
            pass
    owned.clear()


def alignment(pointer: int) -> int:
    """The largest power of two up to 256 that divides a device address."""
    return min(256, pointer & -pointer) if pointer else 256


def alignments(operands: Operands | None) -> tuple[int, ...]:
    if operands is None:
        return ()
    return tuple(alignment(t.pointer) if t is not None else 0
                 for t in (operands.a, operands.b, operands.out, operands.bias))


class Session(threading.local):
    """One hipBLASLt handle and plan cache per thread."""

    def __init__(self) -> None:
        self.handle: int | None = None
        self.plans: dict[tuple, Plan] = {}

    def plan(self, problem: Problem, operands: Operands | None = None) -> Plan:
        """The plan of `problem` for operands of these pointer alignments. As the reference's cuBLASLt adapter keys
        its plans (lib_cublaslt.py:110-135 `PlanKey.alignments`), an algorithm chosen for aligned operands is never
        replayed on less aligned ones. hipBLASLt's preference attributes have no minimum-alignment entries (only
        search mode and workspace size, hipblaslt.h `hipblasLtMatmulPreferenceAttributes_t`), so the key is what
        carries the alignment."""
        if self.handle is None:
            handle = c_void_p()
            api()("hipblasLtCreate", byref(handle))
            self.handle = handle.value
            weakref.finalize(self, api().raw, "hipblasLtDestroy", c_void_p(handle.value))
        key = (problem.dtypes, problem.shape, problem.epilogue, alignments(operands))
        if key not in self.plans:
            self.plans[key] = Plan(self.handle, problem)
        return self.plans[key]


_session = Session()


class HipblasLt(Candidate):
    name, op, origin = "hipblaslt", Op.MATMUL, Origin.VENDOR

    def unavailable(self, target=None) -> str | None:
        try:
            api()
        except LibraryNotFound as error:
            return str(error)
        return None

    def refusal(self, problem: Problem, target=None) -> str | None:
        return refusal(problem)

    def run(self, problem: Problem, operands: Operands, stream: Stream) -> None:
        plan = _session.plan(problem, operands)
        plan.enqueue(_session.handle, operands, stream)
        stream.note("lib.matmul hipblaslt", (operands.a, operands.b, operands.out, operands.bias))


CANDIDATE = HipblasLt()

"""The AMD backend of the runtime contract: gfx950 devices, streams, events, tensors and tile-kernel launches.

`MODULES["amd"]` names this module (reference src/krn/runtime/api.py:321-326, where the module was missing); it
exposes `BACKEND`. Host code is Python over ctypes: the HIP runtime (`libamdhip64`) for memory, streams and events,
the kernel library `libkrn_amd.so` for the hand-written MFMA kernels, and hiprtc plus the HIP module API for tile
programs the generic lowering compiles. The shape follows the CUDA backend of the reference
(src/krn/runtime/cuda_backend.py): a tensor owns its allocation, a launch plans once per signature, an event is settled
by a waiter thread, never by a host callback.
"""

import asyncio
import ctypes
import hashlib
import inspect
import os
import threading
import time
import weakref
from collections import deque
from collections.abc import Callable, Sequence
from ctypes import c_float, c_int, c_int64, c_void_p
from dataclasses import is_dataclass
from pathlib import Path

import numpy as np

from krn_amd import dtypes as D
from krn_amd.compiler import cdna4, dataflow, hipgen, space
from krn_amd.compiler import ir
from krn_amd.compiler.capture import TargetError, capture
from krn_amd.dtypes import Dtype
from krn_amd.frontend import Blocks, Kernel, Tensor, const_fields
from krn_amd.runtime import api, hipapi, library, roctx
from krn_amd.runtime.api import Backend, Bound, Device, Event, Graph, Launcher, Stream, current_stream

TARGET = "gfx950"
HIPRTC_OPTIONS = [f"--offload-arch={TARGET}", "-O3", "-std=c++17", "-ffp-contract=off"]


class HIPEvent(Event):
    """A hipEvent recorded on a stream. Completion is observed by a waiter thread that blocks in
    hipEventSynchronize, so subscribers run on that thread."""

    def __init__(self, device: "HIPDevice", handle: int) -> None:
        self.device, self.handle = device, handle
        self._callbacks: list[Callable[[], None]] = []
        self._done = False
        self._error: BaseException | None = None
        self._lock = threading.Lock()
        self._thread: threading.Thread | None = None

    def done(self) -> bool:
        if self._done:
            return True
        code = hipapi.api().lib.hipEventQuery(c_void_p(self.handle))
        if code == 0:
            self._done = True
        elif code != 600:  # hipErrorNotReady
            self._done, self._error = True, hipapi.HIPError("hipEventQuery", code, "error", "device work failed")
        return self._done

    def wait(self, timeout: float | None = None) -> None:
        """Block until the event completes; with a timeout, poll until the deadline and raise TimeoutError after it
        (reference runtime/cuda_backend.py:132-142)."""
        if timeout is not None:
            deadline = time.monotonic() + timeout
            while not self.done():
                if time.monotonic() > deadline:
                    raise TimeoutError(f"event not completed after {timeout} seconds")
                time.sleep(1e-4)
            return
        try:
            hipapi.api().hipEventSynchronize(c_void_p(self.handle))
        except hipapi.HIPError as error:
            self._error = error
        self._done = True

    def _waiter(self) -> None:
        self.wait()
        with self._lock:
            callbacks, self._callbacks = self._callbacks, []
        for callback in callbacks:
            callback()

    def subscribe(self, callback: Callable[[], None]) -> bool:
        with self._lock:
            if self._done:
                return True
            self._callbacks.append(callback)
            if self._thread is None:
                self._thread = threading.Thread(target=self._waiter, daemon=True)
                self._thread.start()
        return False

    @property
    def error(self) -> BaseException | None:
        return self._error

    def elapsed_since(self, earlier: Event) -> float:
        if not isinstance(earlier, HIPEvent):
            raise TypeError("elapsed time is measured between two HIP events")
        return hipapi.elapsed_ms(earlier.handle, self.handle)

    def __del__(self) -> None:
        try:
            if self._thread is None or not self._thread.is_alive():
                hipapi.api().lib.hipEventDestroy(c_void_p(self.handle))
        except Exception:
            pass


KEEP_LIMIT = 256  # launches a stream holds before it records a marker of its own (reference completion.py:19)


class HIPStream(Stream):
    """An in-order queue of device work. A launch's arguments are held until a marker event recorded after it has
    completed (the `Keeper` of reference runtime/completion.py:99-131): `record()` closes the open launches under its
    event and releases every older marker that is done, and after KEEP_LIMIT unmarked launches the stream records a
    marker itself, so a loop that never synchronizes holds a bounded number of them."""

    def __init__(self, device: "HIPDevice", handle: int) -> None:
        self.device, self.handle = device, handle
        self._open: list[tuple[str, tuple[object, ...]]] = []
        self._marks: deque[tuple[HIPEvent, list[tuple[str, tuple[object, ...]]]]] = deque()

    @property
    def capturing(self) -> bool:
        return hipapi.capturing(self.handle)

    def record(self) -> HIPEvent:
        event = HIPEvent(self.device, hipapi.event_create())
        hipapi.api().hipEventRecord(c_void_p(event.handle), c_void_p(self.handle))
        if not self.capturing:  # a capture's events cannot be queried; the graph holds what it recorded
            self._mark(event)
        return event

    def _mark(self, event: HIPEvent) -> None:
        self._marks.append((event, self._open))
        self._open = []
        while self._marks and self._marks[0][0].done():
            self._marks.popleft()

    def wait(self, event: Event) -> None:
        if not isinstance(event, HIPEvent):
            raise TypeError("a HIP stream waits for HIP events")
        hipapi.api().hipStreamWaitEvent(c_void_p(self.handle), c_void_p(event.handle), 0)

    def pending_launches(self) -> tuple[str, ...]:
        """The launches queued on this stream that have not completed, oldest first: those under markers not yet
        done, then those not yet under a marker (reference api.py:117-118)."""
        marked = [name for event, launches in self._marks if not event.done() for name, _ in launches]
        return (*marked, *(name for name, _ in self._open))

    def note(self, name: str, keep: tuple[object, ...]) -> None:
        """Hold a launch's arguments until the work that reads them has completed."""
        self._open.append((name, keep))
        if len(self._open) >= KEEP_LIMIT and not self.capturing:
            self.record()

    def take(self) -> list[tuple[object, ...]]:
        """Everything held for the launches not yet under a marker, handed over (to a graph that recorded them)."""
        held = [keep for _, keep in self._open]
        self._open = []
        return held

    def sync(self) -> None:
        hipapi.api().hipStreamSynchronize(c_void_p(self.handle))
        self._open = []
        self._marks.clear()


class HIPTensor(Tensor):
    """C-contiguous device memory with its element type (bf16 as uint16 words, fp8 as uint8 codes) and shape.

    Memory is stream ordered (reference runtime/cuda_backend.py module doc and 205-248): a tensor is allocated from
    the device's pool on the stream that was current when it was made, and returned to the pool on that same
    stream when its last reference goes, so the free waits for the work queued there before it. Work on another
    stream reaches the tensor after waiting for an event of the allocating stream, and the launches there hold
    their arguments until they have completed. A tensor made while its stream records a graph is a plain
    allocation that the graph owns, freed with hipFree."""

    def __init__(self, device: "HIPDevice", pointer: int, dtype: Dtype, shape: tuple[int, ...], owner=None,
                 stream: "HIPStream | None" = None) -> None:
        self.device, self.pointer, self.dtype, self.shape = device, pointer, dtype, tuple(int(s) for s in shape)
        self.numpy = D.NUMPY[dtype]
        self._owner = owner  # a view keeps the owner alive; an owner frees its memory
        self._stream = stream  # the allocating stream (stream-ordered memory), or None for a plain allocation
    @property
    def nbytes(self) -> int:
        return self.numpy.itemsize * int(np.prod(self.shape))

    def to_host(self, stream: HIPStream | None = None) -> np.ndarray:
        """A numpy copy, after the work queued on `stream` (default: the current stream) has run."""
        stream = stream or self.device.launch_stream()
        array = np.empty(self.shape, self.numpy)
        if array.nbytes:
            hipapi.api().hipMemcpyAsync(c_void_p(array.ctypes.data), c_void_p(self.pointer), array.nbytes,
                                        hipapi.D2H, c_void_p(stream.handle))
        stream.sync()
        return array

    def copy_from(self, array: np.ndarray, stream: HIPStream | None = None) -> None:
        stream = stream or self.device.launch_stream()
        data = np.ascontiguousarray(array, dtype=self.numpy)
        if data.shape != self.shape:
            raise ValueError(f"shape {data.shape} does not match the tensor's {self.shape}")
        if data.nbytes:
            hipapi.api().hipMemcpyAsync(c_void_p(self.pointer), c_void_p(data.ctypes.data), data.nbytes, hipapi.H2D,
                                        c_void_p(stream.handle))
        stream.sync()

    def __repr__(self) -> str:
        return f"HIPTensor({self.dtype}{list(self.shape)} at {self.pointer:#x})"

    def __del__(self) -> None:
        if self._owner is None and self.pointer:
            try:
                if self._stream is not None:
                    hipapi.free_async(self.pointer, self._stream.handle)
                else:
                    hipapi.free(self.pointer)
            except Exception:
                pass
            self.pointer = 0


def _kind(argument: object) -> object:
    """What compiling depends on in one argument."""
    if isinstance(argument, HIPTensor):
        return ("tensor", argument.dtype, len(argument.shape))
    if is_dataclass(argument) and not isinstance(argument, type):
        return ("config", type(argument).__name__, tuple(sorted(const_fields(argument).items())))
    return ("scalar", type(argument).__name__)


class Program:
    """A hiprtc-compiled module with one entry point."""

    def __init__(self, source: str, entry: str, scratch: int = 0) -> None:
        self.source, self.entry, self.scratch = source, entry, scratch
        self.code = hipapi.rtc().compile(source, entry, HIPRTC_OPTIONS)
        module = c_void_p()
        buffer = ctypes.create_string_buffer(self.code, len(self.code))
        hipapi.api().hipModuleLoadData(ctypes.byref(module), buffer)
        function = c_void_p()
        hipapi.api().hipModuleGetFunction(ctypes.byref(function), module, entry.encode())
        self.module, self.function, self._buffer = module, function, buffer

    @staticmethod
    def table(params: list) -> ctypes.Array:
        """The kernelParams table of `params`: the address of each. The table holds the parameter objects too, so
        the addresses stay valid for as long as the table does."""
        table = (c_void_p * max(len(params), 1))(*(ctypes.addressof(p) for p in params))
        table.params = list(params)
        return table

    def launch(self, grid: tuple[int, int, int], threads: int, table: ctypes.Array, stream: int) -> None:
        hipapi.api().hipModuleLaunchKernel(self.function, grid[0], grid[1], grid[2], threads, 1, 1, 0,
                                           c_void_p(stream), table, None)


_programs: dict[str, Program] = {}
_programs_lock = threading.Lock()


def generic_program(kernel: ir.Kernel) -> Program:
    entry = f"krn_{kernel.name}"
    source, scratch = hipgen.emit(kernel, entry)
    digest = hashlib.sha256(source.encode()).hexdigest()
    with _programs_lock:
        if digest not in _programs:
            _programs[digest] = Program(source, entry, scratch)
        return _programs[digest]


class Launch:
    """One planned launch of one signature: the captured IR, its gfx950 plan, and how to run it."""

    def __init__(self, kernel: ir.Kernel, plan) -> None:
        self.kernel, self.plan = kernel, plan

    def prepare(self, values: list[object], grid: Blocks) -> Callable[[HIPStream], None]:
        """The launch of these argument values on this grid as one call per stream: the plan's checks and argument
        marshalling run here, once, so a `Bound` replays only the library call."""
        call = self.specialised(values, grid)
        route = type(self.plan).__name__
        if call is None:
            call, route = self._generic(values, grid), "GenericPlan"

        name = f"krn:{self.kernel.name} {route}"

        def run(stream: HIPStream) -> None:
            if not roctx.launch_ranges():
                call(stream)
                return
            with roctx.span(name):
                call(stream)

        return run

    def run(self, values: list[object], grid: Blocks, stream: HIPStream) -> None:
        self.prepare(values, grid)(stream)

    def specialised(self, values: list[object], grid: Blocks) -> Callable[[HIPStream], None] | None:
        """The hand-written kernel's call when the plan is one and these arguments and this grid are the whole
        problem it computes; None sends the launch to the generic lowering, which keeps the program's meaning."""
        params = dict(zip((name for name, _ in self.kernel.params), values))
        plan = self.plan
        if isinstance(plan, cdna4.GemmPlan):
            return self._gemm(plan, params, grid)
        if isinstance(plan, cdna4.AttentionPlan):
            return self._attention(plan, params, grid)
        if isinstance(plan, cdna4.SoftmaxPlan):
            return self._softmax(plan, params, grid)
        return None

    def _gemm(self, plan: cdna4.GemmPlan, params: dict, grid: Blocks):
        a, b, c = params[plan.a], params[plan.b], params[plan.c]
        m, k = a.shape
        n = b.shape[0] if plan.layout == "nt" else b.shape[1]
        kb = b.shape[1] if plan.layout == "nt" else b.shape[0]
        extent = space.extent(plan.loop_extent, params) if isinstance(plan.loop_extent, ir.Dim) else None
        if extent != k or kb != k or c.shape != (m, n) or (grid.x, grid.y, grid.z) != (
                -(-n // plan.bn), -(-m // plan.bm), 1):
            return None  # not the whole product: the generic lowering keeps the program's exact meaning
        if len(plan.ops) > library.MAX_OPS:
            return None  # longer epilogue chains than the library's: the generic lowering runs them
        ops = []
        for op in plan.ops:
            if op.op in library.ACTIVATIONS:
                ops.append((library.ACTIVATIONS[op.op], 0.0, 0))
                continue
            base = library.MUL_SCALAR if op.op == "mul" else library.ADD_SCALAR
            if op.tensor is None:
                ops.append((base, float(_scalar_value(op.scalar, params)), 0))
            else:
                vector = params[op.tensor]
                wants = [(m, 1)] if op.axis == "row" else [(1, n), (n,)]
                if vector.shape not in wants or vector.dtype not in library.VECTOR_KINDS:
                    return None
                code = base + (1 if op.axis == "row" else 2) + library.VECTOR_KINDS[vector.dtype]
                ops.append((code, 0.0, vector.pointer))
        if plan.layout == "nn":
            need = library.gemm_nn_workspace_for(a.pointer, b.pointer, m, n, k)
            if need == 0:  # B is read K x N as it lies: no workspace
                direct = library.gemm_nn_call(plan.operand, a.pointer, b.pointer, c.pointer, plan.output, m, n, k,
                                              ops, 0, 0)
                return lambda stream: direct(stream.handle)
            scratch = StreamScratch(need)
            products: dict[int, Callable[[int], None]] = {}  # workspace pointer -> the product marshalled for it

            def nn(stream: HIPStream) -> None:
                workspace = scratch.on(stream)
                product = products.get(workspace.pointer)
                if product is None:
                    product = products[workspace.pointer] = library.gemm_nn_call(
                        plan.operand, a.pointer, b.pointer, c.pointer, plan.output, m, n, k, ops, workspace.pointer,
                        max(need, 1))
                product(stream.handle)
                stream.note(self.kernel.name, (workspace,))

            return nn
        product = library.gemm_nt_call(plan.operand, a.pointer, b.pointer, c.pointer, plan.output, m, n, k, ops)
        return lambda stream: product(stream.handle)

    def _attention(self, plan: cdna4.AttentionPlan, params: dict, grid: Blocks):
        q, k, v, o = (params[n] for n in (plan.q, plan.k, plan.v, plan.o))
        if len(q.shape) != plan.rank:
            return None
        # (batch, heads, seq, d) tensors are C-contiguous, so they are (batch * heads, seq, d) to the kernel
        *lead, sq, d = q.shape
        sk = k.shape[-2]
        bh = int(np.prod(lead))
        if d != plan.d or k.shape != (*lead, sk, d) or v.shape != (*lead, sk, d) or o.shape != (*lead, sq, d):
            return None
        want = (-(-sq // plan.bq), lead[0], 1) if plan.rank == 3 else (-(-sq // plan.bq), lead[1], lead[0])
        if (grid.x, grid.y, grid.z) != want or sk == 0:
            return None
        value = dataflow.scalar_value(plan.scale, params)
        if value is None:
            return None
        # exp(x) is exp2(x * log2(e)): the kernel's exponent scale carries the base
        scale = float(np.float32(float(value) * plan.base))
        return lambda stream: library.attention_fwd(plan.dtype, q.pointer, k.pointer, v.pointer, o.pointer, bh, sq,
                                                    sk, d, scale, plan.causal, stream.handle)

    def _softmax(self, plan: cdna4.SoftmaxPlan, params: dict, grid: Blocks):
        x, y = params[plan.x], params[plan.y]
        if x.shape != y.shape or (grid.x, grid.y, grid.z) != (-(-x.shape[0] // plan.rows), 1, 1):
            return None  # not one block per row group over the whole tensor: the generic lowering keeps its meaning
        rows, cols = x.shape
        width = cols if plan.long_rows else min(cols, plan.cols)
        return lambda stream: library.softmax_rows(plan.dtype, x.pointer, y.pointer, rows, width, cols, cols,
                                                   stream.handle)

    def _generic(self, values: list[object], grid: Blocks) -> Callable[[HIPStream], None]:
        """The hiprtc program of this kernel, compiled (or found) once, with its kernelParams table built once."""
        program = generic_program(self.kernel)
        params: list = []
        for (name, kind), value in zip(self.kernel.params, values):
            if isinstance(kind, ir.TensorType):
                if not isinstance(value, HIPTensor) or len(value.shape) != kind.rank:
                    raise TypeError(f"{self.kernel.name}: `{name}` needs a rank-{kind.rank} device tensor")
                params.append(c_void_p(value.pointer))
                params.extend(c_int64(s) for s in value.shape)
            elif kind.is_float:
                params.append(ctypes.c_double(value) if kind.bits == 64 else c_float(value))
            elif kind.bits == 64:
                params.append(c_int64(int(value)))
            elif kind.bits == 8:
                params.append(ctypes.c_uint8(int(value)) if kind.kind.value == "uint" else ctypes.c_int8(int(value)))
            else:
                params.append(c_int(int(value)))
        dims = (grid.x, grid.y, grid.z)
        blocks = grid.x * grid.y * grid.z
        if blocks == 0:
            return lambda stream: None  # a zero-extent grid launches nothing (reference cuda_backend.py:377-383)
        if not program.scratch:
            table = Program.table(params)
            return lambda stream: program.launch(dims, hipgen.THREADS, table, stream.handle)
        scratch = StreamScratch(blocks * program.scratch)
        slot = c_void_p(0)
        table = Program.table([*params, slot])

        def run(stream: HIPStream) -> None:
            memory = scratch.on(stream)
            slot.value = memory.pointer
            program.launch(dims, hipgen.THREADS, table, stream.handle)
            stream.note(self.kernel.name, (memory,))

        return run


class StreamScratch:
    """Device scratch of one prepared launch, one buffer per stream it runs on: launches on one stream run in order,
    so every replay there reuses that stream's buffer, allocated (stream ordered) on its first use. The prepared
    launch (a `Bound`, a graph) owns it; each launch also holds its buffer until the launch completes."""

    def __init__(self, nbytes: int) -> None:
        self.nbytes = max(nbytes, 1)
        self._buffers: dict[int, HIPTensor] = {}

    def on(self, stream: HIPStream) -> HIPTensor:
        buffer = self._buffers.get(stream.handle)
        if buffer is None:
            buffer = self._buffers[stream.handle] = stream.device.empty_on(stream, D.U8, self.nbytes)
        return buffer


def _scalar_value(e: ir.Expr, params: dict) -> np.float32:
    """A float32 scalar epilogue operand, evaluated as the kernel would: each operation rounded to float32."""
    match e:
        case ir.Const(value=v):
            return np.float32(v)
        case ir.Param(name=n):
            return np.float32(params[n])
        case ir.Cast(operand=o):
            return np.float32(_scalar_value(o, params))
        case ir.Binary(op=op, lhs=a, rhs=b):
            x, y = _scalar_value(a, params), _scalar_value(b, params)
            with np.errstate(all="ignore"):
                return np.float32({ir.Op.MUL: np.multiply, ir.Op.ADD: np.add, ir.Op.SUB: np.subtract,
                                   ir.Op.DIV: np.divide}[op](x, y))
    raise ValueError(f"{type(e).__name__} is not a scalar epilogue operand")


def _blocks(launch: object) -> Blocks | None:
    """An explicit grid from any geometry object with the reference's public fields (src/krn/frontend/geometry.py:
    8-43): `Tiles` (`shape`, `tile`, `.blocks`) or `Blocks` (`x`, `y`, `z`, `threads`). `Items` launches one thread
    per item, which a tile program does not: it is refused."""
    if launch is None or isinstance(launch, Blocks):
        return launch
    if hasattr(launch, "blocks"):
        launch = launch.blocks
    if all(hasattr(launch, axis) for axis in ("x", "y", "z")):
        return Blocks(int(launch.x), int(launch.y), int(launch.z), getattr(launch, "threads", None))
    raise TargetError(f"{type(launch).__name__} geometry", TARGET, "it is not a tile launch geometry (one thread per "
                      "item is not how a tile program runs)", "launch with Blocks or Tiles")


_plans: dict[tuple, Launch] = {}  # (kernel, argument kinds) -> its captured IR and plan
_plans_lock = threading.Lock()


class HIPLauncher(Launcher):
    """A kernel with an optional explicit geometry. The first call of a signature captures and plans it."""

    def __init__(self, device: "HIPDevice", kernel: Kernel, launch: object = None) -> None:
        # only `fn` and `name` are read, as the reference's SourceLauncher does (src/krn/runtime/runtime.py:463-470),
        # so krn's own Kernel objects launch here unchanged
        self.device, self.kernel, self.launch = device, kernel, _blocks(launch)
        self.parameters = tuple(inspect.signature(kernel.fn).parameters)

    def ordered(self, args: tuple, kwargs: dict) -> tuple:
        if not kwargs and len(args) == len(self.parameters):
            return args
        try:
            ordered = (*args, *(kwargs.pop(name) for name in self.parameters[len(args):]))
        except KeyError as missing:
            raise TypeError(f"{self.kernel.name}() is missing the argument {missing}") from None
        if kwargs or len(ordered) != len(self.parameters):
            raise TypeError(f"{self.kernel.name}() takes {len(self.parameters)} arguments")
        return ordered

    def plan(self, args: Sequence[object]) -> Launch:
        # launchers are made per call (`k(..., launch=...)`, `k[config]`): the plans live with the process
        signature = (self.kernel, *map(_kind, args))
        try:
            return _plans[signature]
        except KeyError:
            pass
        with _plans_lock:
            if signature not in _plans:
                consts = {n: const_fields(a) for n, a in zip(self.parameters, args)
                          if is_dataclass(a) and not isinstance(a, type)}
                dtypes = {n: a.dtype for n, a in zip(self.parameters, args) if isinstance(a, HIPTensor)}
                path = Path(inspect.getsourcefile(self.kernel.fn))
                kernel = capture(path, self.kernel.name, consts=consts, dtypes=dtypes)
                _plans[signature] = Launch(kernel, cdna4.lower(kernel))
            return _plans[signature]

    def encode(self, args: tuple) -> Callable[[HIPStream], None]:
        launch = self.plan(args)
        values = space.runtime_args(launch.kernel, args)
        grid = self.launch if self.launch is not None else space.geometry(launch.kernel, values)

        call = launch.prepare(values, grid)
        keep = tuple(values)

        def run(stream: HIPStream) -> None:
            call(stream)
            stream.note(self.kernel.name, keep)

        return run

    def __call__(self, *args, **kwargs) -> None:
        self.encode(self.ordered(args, kwargs))(self.device.launch_stream())

    def submit(self, *args, **kwargs) -> HIPEvent:
        stream = self.device.launch_stream()
        self.encode(self.ordered(args, kwargs))(stream)
        return stream.record()

    def bind(self, *args, **kwargs) -> "HIPBound":
        return HIPBound(self, self.ordered(args, kwargs))

    def explain(self, *args, **kwargs) -> dict:
        """What a launch with these arguments runs: the plan that serves it and, for the generic lowering, why no
        hand-written kernel took it and how each product runs ("mfma 16x16x16 bf16" or "scalar fma")."""
        args = self.ordered(args, kwargs)
        launch = self.plan(args)
        values = space.runtime_args(launch.kernel, args)
        grid = self.launch if self.launch is not None else space.geometry(launch.kernel, values)
        if launch.specialised(values, grid) is not None:
            return {"kernel": launch.kernel.name, "target": TARGET, "plan": type(launch.plan).__name__,
                    "detail": repr(launch.plan)}
        if isinstance(launch.plan, cdna4.GenericPlan):
            why = cdna4.why_generic(launch.kernel)
        else:
            why = [f"the program is a {type(launch.plan).__name__}, but these arguments or this grid are not the whole "
                   "problem its kernel computes (the grid must cover the output once, the loop the whole extent)"]
        return {"kernel": launch.kernel.name, "target": TARGET, "plan": "GenericPlan", "detail": "hipgen",
                "products": hipgen.products(launch.kernel), "why": why}


class HIPBound(Bound):
    def __init__(self, launcher: HIPLauncher, args: tuple) -> None:
        self.launcher = launcher
        self.rebind(*args)

    def rebind(self, *args, **kwargs) -> None:
        self.run = self.launcher.encode(self.launcher.ordered(args, kwargs))

    def __call__(self) -> None:
        self.run(self.launcher.device.launch_stream())

    def submit(self) -> HIPEvent:
        stream = self.launcher.device.launch_stream()
        self.run(stream)
        return stream.record()


class HIPGraph(Graph):
    """The launches of one function captured from a stream into a hipGraph and replayed with one hipGraphLaunch
    (reference runtime/cuda_backend.py:486-551, `CUDAGraph`). A replay needs the recorded arguments (the same
    objects): the recorded nodes keep their pointers, so new arguments raise TargetError; tensor contents may change
    between replays. Scratch memory that a recorded launch allocated lives as long as the graph. With
    KRN_GRAPHS=0 the function is instead called again on every replay (plain launches)."""

    def __init__(self, device: "HIPDevice", fn: Callable, args: tuple, kwargs: dict) -> None:
        self.device, self._fn, self._recorded = device, fn, (args, kwargs)
        self._executable: int | None = None
        self._keep: list[tuple[object, ...]] = []
        if os.environ.get("KRN_GRAPHS", "1") != "0":
            self._executable = self._capture(*args, **kwargs)

    def __call__(self, *args, **kwargs) -> None:
        recorded_args, recorded_kwargs = self._recorded
        same = (len(args) == len(recorded_args) and all(a is b for a, b in zip(args, recorded_args))
                and kwargs.keys() == recorded_kwargs.keys()
                and all(kwargs[name] is recorded_kwargs[name] for name in kwargs))
        if self._executable is not None and same:
            stream = self.device.launch_stream()
            hipapi.api().hipGraphLaunch(c_void_p(self._executable), c_void_p(stream.handle))
            stream.note("graph", (self,))
            return
        if self._executable is not None:
            raise TargetError("graph replay", self.device.arch,
                              "hipGraph nodes keep their recorded arguments; krn does not patch node parameters",
                              "record a new graph for these arguments or set KRN_GRAPHS=0")
        self._fn(*args, **kwargs)

    def submit(self, *args, **kwargs) -> HIPEvent:
        self(*args, **kwargs)
        return self.device.launch_stream().record()

    def _capture(self, *args, **kwargs) -> int:
        stream = self.device.capture_stream()
        handle = c_void_p(stream.handle)
        hipapi.api().hipStreamBeginCapture(handle, hipapi.CAPTURE_RELAXED)
        graph = c_void_p()
        try:
            with stream:
                self._fn(*args, **kwargs)
        except BaseException:  # end the capture and drop its graph, then report the original error
            if hipapi.api().raw("hipStreamEndCapture", handle, ctypes.byref(graph)) == 0 and graph.value:
                hipapi.api().raw("hipGraphDestroy", graph)
            stream.take()
            raise
        hipapi.api().hipStreamEndCapture(handle, ctypes.byref(graph))
        executable = c_void_p()
        try:
            hipapi.api().hipGraphInstantiate(ctypes.byref(executable), graph, None, None, 0)
        except BaseException:
            hipapi.api().raw("hipGraphDestroy", graph)
            raise
        # what the recorded launches hold (scratch tensors, arguments) now lives with the graph
        self._keep = stream.take()
        weakref.finalize(self, _release_graph, executable.value, graph.value)
        return executable.value


def _release_graph(executable: int, graph: int) -> None:
    try:
        hipapi.api().raw("hipGraphExecDestroy", c_void_p(executable))
        hipapi.api().raw("hipGraphDestroy", c_void_p(graph))
    except Exception:
        pass


class HIPDevice(Device):
    """One gfx950 GPU."""

    def __init__(self, arch: str, ordinal: int = 0) -> None:
        if hipapi.device_count() == 0:
            raise api.BackendUnavailable("no HIP device is visible to this process")
        self.arch, self.ordinal = arch, ordinal
        hipapi.api().hipSetDevice(ordinal)
        library.lib()  # the kernel library must be present: there is no fallback path
        hipapi.keep_pool(ordinal)
        self._default = HIPStream(self, hipapi.stream_create())
        self._streams: list[HIPStream] = [self._default]

    @property
    def default_stream(self) -> HIPStream:
        return self._default

    def launch_stream(self) -> HIPStream:
        stream = current_stream.get()
        return stream if isinstance(stream, HIPStream) else self._default

    def stream(self) -> HIPStream:
        created = HIPStream(self, hipapi.stream_create())
        self._streams.append(created)
        return created

    def capture_stream(self) -> HIPStream:
        """The stream graphs are recorded on (one per device, reused)."""
        if getattr(self, "_capture", None) is None:
            self._capture = self.stream()
        return self._capture

    def empty(self, dtype, *shape: int) -> HIPTensor:
        """Uninitialized memory, allocated on the launch stream (stream ordered) or, while that stream records a
        graph, by a plain allocation the graph keeps."""
        return self.empty_on(self.launch_stream(), dtype, *shape)

    def empty_on(self, stream: HIPStream, dtype, *shape: int) -> HIPTensor:
        element = D.of(dtype)
        count = int(np.prod(shape)) if shape else 1
        nbytes = count * D.NUMPY[element].itemsize
        if stream.capturing:
            return HIPTensor(self, hipapi.malloc(nbytes), element, shape)
        return HIPTensor(self, hipapi.malloc_async(nbytes, stream.handle), element, shape, stream=stream)

    def to_device(self, array: np.ndarray, dtype=None) -> HIPTensor:
        """A device copy of a host array. bf16 and fp8 arrays pass their element type (`T.bf16`, `T.f8e4m3fn`)."""
        array = np.ascontiguousarray(array)
        element = D.of(dtype) if dtype is not None else D.FROM_NUMPY[array.dtype]
        if array.dtype != D.NUMPY[element]:
            raise TypeError(f"a {element} tensor is stored as {D.NUMPY[element]}, got {array.dtype}")
        tensor = self.empty(element, *array.shape)
        tensor.copy_from(array)
        return tensor

    def launcher(self, kernel: Kernel, launch=None) -> HIPLauncher:
        return HIPLauncher(self, kernel, launch)

    def graph(self, fn: Callable, *args, **kwargs) -> HIPGraph:
        return HIPGraph(self, fn, args, kwargs)

    def sync(self) -> None:
        for stream in self._streams:
            stream.sync()

    async def synchronize(self) -> None:
        await asyncio.get_running_loop().run_in_executor(None, self.sync)


class HIPBackend(Backend):
    vendor = "amd"

    def __init__(self) -> None:
        self._devices: dict[str, HIPDevice] = {}
        self._lock = threading.Lock()

    def device(self, target) -> HIPDevice:
        """The one device of `target`: krn's `Target` (an AMD target, read by its `arch`; reference
        src/krn/runtime/api.py:312-354, src/krn/facts/targets.py:214-237) or the arch name itself."""
        arch = api.arch_of(target)
        if getattr(target, "vendor", self.vendor) != self.vendor:
            raise TypeError(f"the amd backend builds devices for AMD targets, not {arch}")
        if arch != TARGET:
            raise api.BackendUnavailable(f"the AMD backend serves {TARGET}, not {arch}")
        with self._lock:
            if arch not in self._devices:
                self._devices[arch] = HIPDevice(arch)
            return self._devices[arch]


BACKEND = HIPBackend()

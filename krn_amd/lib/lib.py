"""`lib.matmul` on gfx950: one operation, an ordered list of candidates, and a dispatcher that takes the first one
that accepts the problem (reference src/krn/lib/lib.py:182-264 `Problem`/`Candidate`/`PREFERENCE`, 548-615
`matmul`).

The AMD order is the reference's own, `("hipblaslt", "ours", "host")` (lib.py:264): the vendor library first, then
krn's tile program (`lib_ours`), then the host. This build has no host candidate: nothing here computes on the CPU,
so it is listed as unavailable and a problem every device candidate refuses raises `NoCandidate` with each reason.
A candidate may also decline at run time, before it enqueues anything (hipBLASLt finding no algorithm), and the
call falls to the next one.
"""

import os
from abc import ABC, abstractmethod
from dataclasses import dataclass
from enum import Enum
from importlib import import_module

from krn_amd.dtypes import BF16, F16, F32, Dtype
from krn_amd.runtime.api import Stream, current_stream, default_device


class Op(str, Enum):
    """Library operations. A `str` enum, as the reference's StrEnum (lib.py:76-79): `Op.MATMUL == "matmul"`."""

    MATMUL = "matmul"

    def __str__(self) -> str:
        return self.value


class Epilogue(str, Enum):
    """What follows the product, in the reference's names (lib.py:82-91 `Epilogue`, a StrEnum): members compare
    equal to their string values, and `matmul(..., epilogue="bias_gelu")` is accepted."""

    NONE = "none"
    BIAS = "bias"
    RELU = "relu"
    GELU = "gelu"
    BIAS_RELU = "bias_relu"
    BIAS_GELU = "bias_gelu"
    SILU = "silu"

    def __str__(self) -> str:
        return self.value

    @property
    def has_bias(self) -> bool:
        return self in (Epilogue.BIAS, Epilogue.BIAS_RELU, Epilogue.BIAS_GELU)


class Origin(Enum):
    VENDOR = "vendor"
    OURS = "ours"


@dataclass(frozen=True)
class Problem:
    """`shape` is (m, n, k); `dtypes` are (a, b, out)."""

    op: Op
    dtypes: tuple[Dtype, Dtype, Dtype]
    shape: tuple[int, int, int]
    epilogue: Epilogue = Epilogue.NONE


@dataclass(frozen=True)
class Operands:
    a: object
    b: object
    out: object
    bias: object | None = None


class Declined(RuntimeError):
    """Raised by `Candidate.run` before it enqueues anything, when planning shows it cannot take the problem after
    all; the call falls to the next candidate and the reason joins the list `NoCandidate` prints."""


class NoCandidate(LookupError):
    """Every candidate refused; the message lists each refusal."""


class Candidate(ABC):
    """One implementation of one operation. `unavailable` is why it cannot run on this machine at all, `refusal` why
    it does not take this problem; `run` only enqueues, on the given stream, and never synchronizes. The `target`
    arguments mirror the reference's signatures (lib.py:201-235); this build serves gfx950 only and ignores them."""

    name: str
    op: Op
    origin: Origin

    def unavailable(self, target=None) -> str | None:
        return None

    @abstractmethod
    def refusal(self, problem: Problem, target=None) -> str | None: ...

    @abstractmethod
    def run(self, problem: Problem, operands: Operands, stream: Stream) -> None: ...


class Host(Candidate):
    """The reference's last resort computes on the host. krn_amd computes only on the GPU."""

    name, op, origin = "host", Op.MATMUL, Origin.OURS

    def unavailable(self, target=None) -> str | None:
        return "krn_amd has no host path: every product runs on the GPU"

    def refusal(self, problem: Problem, target=None) -> str | None:
        return self.unavailable()

    def run(self, problem: Problem, operands: Operands, stream: Stream) -> None:
        raise Declined(self.unavailable())


PREFERENCE: dict[Op, tuple[str, ...]] = {Op.MATMUL: ("hipblaslt", "ours", "host")}
MODULES = {"hipblaslt": "krn_amd.lib.lib_hipblaslt", "ours": "krn_amd.lib.lib_ours"}


def candidate(name: str) -> Candidate:
    """The candidate called `name` (its adapter module is imported on first use)."""
    if name == "host":
        return Host()
    if name not in MODULES:
        raise KeyError(f"unknown matmul candidate {name!r}; known: {', '.join(PREFERENCE[Op.MATMUL])}")
    return import_module(MODULES[name]).CANDIDATE


def order(library: str | None = None) -> tuple[str, ...]:
    """The candidates tried, in order: one named library (the `library=` argument, else `KRN_LIB`), or the
    preference order."""
    chosen = library or os.environ.get("KRN_LIB") or None
    return (chosen,) if chosen else PREFERENCE[Op.MATMUL]


def product_type(a: Dtype, b: Dtype) -> Dtype:
    """The type that holds both inputs: the type itself for two equal ones, float32 otherwise."""
    return a if a == b else F32


FLOATS = (F16, BF16, F32)


def matmul(a, b, *, epilogue: Epilogue = Epilogue.NONE, bias=None, out=None, library: str | None = None):
    """`a @ b` with an optional fused epilogue, enqueued on the current stream; returns `out`, allocated when not
    given (reference lib.py:581-615). `library` names one candidate instead of the preference order."""
    epilogue = Epilogue(epilogue)
    if len(a.shape) != 2 or len(b.shape) != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"matmul needs (m, k) @ (k, n) matrices, got {a.shape} @ {b.shape}")
    if epilogue.has_bias and (bias is None or tuple(bias.shape) != (b.shape[1],)):
        raise ValueError(f"{epilogue.value} needs a bias vector of length {b.shape[1]}")
    result_type = out.dtype if out is not None else product_type(a.dtype, b.dtype)
    if epilogue.has_bias and bias.dtype != result_type:
        # the bias is a vector of the output type (reference lib.py:576-590 `Vector[Y]`); every candidate reads it so
        raise ValueError(f"{epilogue.value} needs a {result_type} bias (the output type), got {bias.dtype}")
    device = default_device()
    stream = current_stream.get() or device.default_stream
    if out is not None and tuple(out.shape) != (a.shape[0], b.shape[1]):
        raise ValueError(f"out has shape {out.shape}, the product {(a.shape[0], b.shape[1])}")
    result = out if out is not None else device.empty(result_type, a.shape[0], b.shape[1])
    problem = Problem(Op.MATMUL, (a.dtype, b.dtype, result.dtype), (a.shape[0], b.shape[1], a.shape[1]), epilogue)
    launch(problem, Operands(a, b, result, bias), stream, library)
    return result


def launch(problem: Problem, operands: Operands, stream: Stream, library: str | None = None) -> str:
    """Run the first candidate that takes the problem; returns its name."""
    reasons = []
    for name in order(library):
        chosen = candidate(name)
        reason = chosen.unavailable() or chosen.refusal(problem)
        if reason is None:
            try:
                chosen.run(problem, operands, stream)
                return name
            except Declined as declined:
                reason = str(declined)
        reasons.append(f"{name}: {reason}")
    raise NoCandidate(f"no matmul candidate takes {problem}:\n  " + "\n  ".join(reasons))


def choice(problem: Problem, library: str | None = None) -> str:
    """The candidate the static order picks for `problem` (without running it)."""
    for name in order(library):
        chosen = candidate(name)
        if (chosen.unavailable() or chosen.refusal(problem)) is None:
            return name
    raise NoCandidate(f"no matmul candidate takes {problem}")

"""ROCTx ranges: named host-side ranges that `rocprofv3 --marker-trace` records on the timeline beside the kernels.

Mirrors the reference's AMD annotation backend (src/krn/profile/providers/amd/tracer.py:31-56, `ROCTxTracer`):
`start(name)` opens a range and returns the exact call that closes it, `is_available()` says whether the library
loads (rocprofiler-sdk's, which rocprofv3 records, else roctracer's libroctx64), and native activity collection is
refused with a `TargetError` as there. Beyond that, `span(name)` is a context manager over `start`, and with `launch_ranges(True)` (or `KRN_ROCTX=1` in the environment) every tile
program launch enqueues inside a range named `krn:<kernel> <plan>`, so a marker trace ties each kernel dispatch to
the program that asked for it.
"""

import os
from collections.abc import Callable, Iterator
from contextlib import contextmanager
from ctypes import c_char_p, c_uint64
from functools import cache
from typing import ClassVar

from krn_amd.compiler.capture import TargetError
from krn_amd.hw import Libraries

Marker = Callable[[], None]

_launch_ranges = os.environ.get("KRN_ROCTX") == "1"


@cache
def _handle():
    handle = Libraries.load("roctx").handle
    handle.roctxRangeStartA.argtypes = [c_char_p]
    handle.roctxRangeStartA.restype = c_uint64
    handle.roctxRangeStop.argtypes = [c_uint64]
    handle.roctxRangeStop.restype = None
    return handle


class ROCTxTracer:
    """ROCTx start/stop ranges (thread-safe: each range has its own id)."""

    vendor: ClassVar[str] = "amd"
    label: ClassVar[str] = "roctx"

    @classmethod
    def is_available(cls) -> bool:
        return Libraries.available("roctx")

    def start(self, name: str) -> Marker:
        """Open a range and return the call that closes exactly it."""
        handle = _handle()
        range_id = handle.roctxRangeStartA(name.encode())
        return lambda: handle.roctxRangeStop(range_id)

    def supported(self):
        raise TargetError("rocprofiler-sdk activity", "AMD", "no native activity collector is built",
                          "use rocprofv3 --kernel-trace / --marker-trace around the program")

    def collect(self, kinds=None):
        return self.supported()


@contextmanager
def span(name: str) -> Iterator[None]:
    """A ROCTx range around the body."""
    close = ROCTxTracer().start(name)
    try:
        yield
    finally:
        close()


def launch_ranges(on: bool | None = None) -> bool:
    """Whether each tile program launch is wrapped in a ROCTx range; `on` switches it."""
    global _launch_ranges
    if on is not None:
        _launch_ranges = bool(on)
    return _launch_ranges

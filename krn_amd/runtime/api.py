"""The host contract of a device backend: devices, streams, events, launchers, bound launches and graphs.

Mirrors `krn.runtime.api` (reference src/krn/runtime/api.py:54-354): every enqueue returns at once; an `Event` is
awaitable; the current stream is a `ContextVar`; a `Launcher` is a kernel bound to a geometry, `bind` marshals once
into a `Bound` fast path; `Device.current()` picks the backend of the selected target. `KRN_TARGET=gfx950` selects
the AMD backend `krn_amd.runtime.hip` (the module `MODULES["amd"]` names).
"""

import asyncio
import os
from abc import ABC, abstractmethod
from collections.abc import Callable
from contextvars import ContextVar
from functools import partial
from importlib import import_module


class Event(ABC):
    """A point in a stream's order. Awaiting it suspends the awaiting task only; `done()` never blocks."""

    @abstractmethod
    def done(self) -> bool: ...

    @abstractmethod
    def subscribe(self, callback: Callable[[], None]) -> bool:
        """Run once on the resolving thread; return True if already resolved without retaining the callback."""

    @property
    @abstractmethod
    def error(self) -> BaseException | None:
        """What the device reported for the work before this event, once it is done."""

    def wait(self, timeout: float | None = None) -> None:
        raise NotImplementedError

    @abstractmethod
    def elapsed_since(self, earlier: "Event") -> float:
        """Milliseconds between two events of one device, by the device clock."""

    def __await__(self):
        loop = asyncio.get_running_loop()
        future = loop.create_future()
        if self.subscribe(partial(self._wake, loop, future)):
            self._deliver(future)
        return future.__await__()

    def _wake(self, loop: asyncio.AbstractEventLoop, future: asyncio.Future) -> None:
        try:
            loop.call_soon_threadsafe(self._deliver, future)
        except RuntimeError:  # the loop closed while its task waited
            pass

    def _deliver(self, future: asyncio.Future) -> None:
        if future.done():
            return
        if (error := self.error) is None:
            future.set_result(None)
        else:
            future.set_exception(error)


current_stream: ContextVar["Stream | None"] = ContextVar("krn_amd_current_stream", default=None)
_tokens: ContextVar[tuple] = ContextVar("krn_amd_stream_tokens", default=())


class Stream(ABC):
    """An in-order queue of device work."""

    device: "Device"

    @property
    def capturing(self) -> bool:
        return False

    @abstractmethod
    def record(self) -> Event: ...

    @abstractmethod
    def wait(self, event: Event) -> None: ...

    @abstractmethod
    def pending_launches(self) -> tuple[str, ...]: ...

    def __enter__(self):
        _tokens.set((*_tokens.get(), current_stream.set(self)))
        return self

    def __exit__(self, *exc: object) -> None:
        *outer, token = _tokens.get()
        current_stream.reset(token)
        _tokens.set(tuple(outer))

    async def __aenter__(self):
        return self.__enter__()

    async def __aexit__(self, *exc: object) -> None:
        self.__exit__(*exc)
        await self.record()


class Launcher(ABC):
    """A kernel bound to a launch geometry. Calling it enqueues on the current stream and returns at once."""

    @abstractmethod
    def __call__(self, *args, **kwargs) -> None: ...

    @abstractmethod
    def submit(self, *args, **kwargs) -> Event: ...

    @abstractmethod
    def bind(self, *args, **kwargs) -> "Bound": ...

    def explain(self, *args, **kwargs) -> dict:
        raise NotImplementedError


class Bound(ABC):
    """A launch whose arguments are already encoded: one driver call, no marshalling."""

    @abstractmethod
    def __call__(self) -> None: ...

    @abstractmethod
    def submit(self) -> Event: ...

    @abstractmethod
    def rebind(self, *args, **kwargs) -> None: ...


class ConfiguredBound(Bound):
    def __init__(self, inner: Bound, config: object) -> None:
        self.inner, self.config = inner, config

    def __call__(self) -> None:
        self.inner()

    def submit(self) -> Event:
        return self.inner.submit()

    def rebind(self, *args, **kwargs) -> None:
        self.inner.rebind(self.config, *args, **kwargs)


class Configured(Launcher):
    """The launcher of a configured kernel: the configuration is passed as the first argument
    (reference src/krn/runtime/api.py:206-222)."""

    def __init__(self, inner: Launcher, config: object) -> None:
        self.inner, self.config = inner, config

    def __call__(self, *args, **kwargs) -> None:
        self.inner(self.config, *args, **kwargs)

    def submit(self, *args, **kwargs) -> Event:
        return self.inner.submit(self.config, *args, **kwargs)

    def bind(self, *args, **kwargs) -> Bound:
        return ConfiguredBound(self.inner.bind(self.config, *args, **kwargs), self.config)

    def explain(self, *args, **kwargs) -> dict:
        return self.inner.explain(self.config, *args, **kwargs)


class Graph(ABC):
    """Recorded launches that replay with one call per graph."""

    @abstractmethod
    def __call__(self, *args, **kwargs) -> None: ...

    @abstractmethod
    def submit(self, *args, **kwargs) -> Event: ...


class Device(ABC):
    """One GPU (or the host), with the target facts the compiler needs."""

    arch: str

    @classmethod
    def current(cls) -> "Device":
        return default_device()

    @property
    @abstractmethod
    def default_stream(self) -> Stream: ...

    @abstractmethod
    def stream(self) -> Stream: ...

    @abstractmethod
    def to_device(self, array, dtype=None): ...

    @abstractmethod
    def empty(self, dtype, *shape: int): ...

    @abstractmethod
    def launcher(self, kernel, launch=None) -> Launcher: ...

    @abstractmethod
    def graph(self, fn: Callable, *args, **kwargs) -> Graph: ...

    @abstractmethod
    async def synchronize(self) -> None: ...


class Backend(ABC):
    """What a vendor implementation provides; its module exposes one instance as `BACKEND`."""

    vendor: str

    @abstractmethod
    def device(self, target) -> Device:
        """The one device of `target`: krn's `Target` (read by `.arch` and `.vendor`) or an arch name."""


MODULES = {"amd": "krn_amd.runtime.hip"}
VENDORS = {"gfx950": "amd"}


class BackendUnavailable(RuntimeError):
    """The target was selected but its backend cannot run here (no module, no library or no device)."""


def target() -> str:
    """The selected target: `KRN_TARGET` (reference src/krn/runtime/settings.py:348-352), gfx950 by default."""
    return os.environ.get("KRN_TARGET", "gfx950")


def arch_of(target) -> str:
    """The arch name of a target: krn's `Target` carries it as `.arch` (reference src/krn/facts/targets.py:99); a
    plain string is the name itself."""
    if isinstance(target, str):
        return target
    arch = getattr(target, "arch", None)
    if not isinstance(arch, str):
        raise TypeError(f"a target is an arch name or an object with an `arch` name, not {type(target).__name__}")
    return arch


def default_device() -> Device:
    return device_of(target())


def device_of(target) -> Device:
    """The one device of `target` (krn's `Target` or its arch name) for this process; the backend module is
    imported on first use (reference src/krn/runtime/api.py:341-354: the vendor names the module, nothing
    registers it)."""
    arch = arch_of(target)
    vendor = getattr(target, "vendor", None) or VENDORS.get(arch)
    return _device(arch, vendor, target)


_devices: dict[tuple[str, str | None], Device] = {}


def _device(arch: str, vendor: str | None, target) -> Device:
    key = (arch, vendor)
    if key in _devices:
        return _devices[key]
    if vendor not in MODULES:
        raise BackendUnavailable(f"target {arch!r} has no backend in krn_amd; set KRN_TARGET=gfx950")
    try:
        backend: Backend = import_module(MODULES[vendor]).BACKEND
    except (ImportError, AttributeError, OSError) as error:
        raise BackendUnavailable(f"{arch} was selected but its backend {MODULES[vendor]!r} failed to load: {error}") \
            from error
    _devices[key] = device = backend.device(target)
    return device

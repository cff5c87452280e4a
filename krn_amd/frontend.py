"""The kernel-language surface of the tile path: `@kernel`, `Tile`, `Tensor`/`Matrix`/`Vector`, `T.*` element types,
`zeros`, `arange`, `where`, `pipelined`, `block`, `@struct`/`Const` and the launch geometries.

These are typed stubs, as in krn (reference src/krn/frontend/memory.py:53-408, kernel.py:22-105, geometry.py:9-39):
a kernel body is never executed in Python. It is captured from its source file (`krn_amd.compiler.capture`) and run
by the device backend. Calling a stub outside a kernel raises.
"""

import inspect
from dataclasses import dataclass, fields, is_dataclass
from typing import Any, Generic, TypeVar, get_origin

from krn_amd import dtypes as _d

V = TypeVar("V")


def _stub(*_: object, **__: object) -> Any:
    raise RuntimeError("tile operations exist only inside a @kernel body, which is captured, not executed")


class _Element:
    """An element type usable in annotations (`Matrix[T.f16]`, `scale: T.f32`) and in `zeros(T.f32, ...)`."""

    dtype_name = ""

    def __init_subclass__(cls, name: str = "", **kwargs: object) -> None:
        super().__init_subclass__(**kwargs)
        cls.dtype_name = name


def _element(name: str) -> type:
    return type(name, (_Element,), {}, name=name)


class T:
    """The element types: `T.f32`, `T.bf16`, `T.f8e4m3fn`, `T.i8`, ..."""

    bool = _element("bool")
    i8, i16, i32, i64 = (_element(n) for n in ("i8", "i16", "i32", "i64"))
    u8, u16, u32, u64 = (_element(n) for n in ("u8", "u16", "u32", "u64"))
    f16, bf16, f32, f64 = (_element(n) for n in ("f16", "bf16", "f32", "f64"))
    f8e4m3fn, f8e5m2 = _element("f8e4m3fn"), _element("f8e5m2")


bool_, i8, i16, i32, i64 = T.bool, T.i8, T.i16, T.i32, T.i64
u8, u16, u32, u64 = T.u8, T.u16, T.u32, T.u64
f16, bf16, f32, f64, f8e4m3fn, f8e5m2 = T.f16, T.bf16, T.f32, T.f64, T.f8e4m3fn, T.f8e5m2


class Tensor(Generic[V]):
    """A row-major view of device memory; slices of it are tiles, scalar indices single elements."""

    shape: tuple[int, ...]

    def __class_getitem__(cls, item: object) -> Any:
        return cls

    def to_host(self) -> Any:
        raise NotImplementedError


Matrix = Tensor
Vector = Tensor


class Tile(Generic[V]):
    """A block-cooperative value of fixed shape; its operations are captured, never executed."""

    def __class_getitem__(cls, item: object) -> Any:
        return cls

    __add__ = __sub__ = __mul__ = __truediv__ = __matmul__ = __neg__ = _stub
    __lt__ = __le__ = __gt__ = __ge__ = _stub
    transpose = to = max = min = sum = mean = exp = exp2 = log = sqrt = maximum = minimum = _stub


class Const(Generic[V]):
    """A compile-time field of a `@struct` configuration: each distinct value is its own specialization."""

    def __class_getitem__(cls, item: object) -> Any:
        return _ConstAlias(item)


@dataclass(frozen=True)
class _ConstAlias:
    of: object


def is_const(annotation: object) -> bool:
    """Whether a field annotation is `Const[...]`: this module's, or krn's own (`type Const[T] = T`, reference
    src/krn/frontend/records.py:17, whose subscript has that alias as its origin), or the same written as a string."""
    origin = get_origin(annotation)
    return isinstance(annotation, _ConstAlias) or origin is Const or getattr(origin, "__name__", None) == "Const" or (
        isinstance(annotation, str) and annotation.startswith("Const[")
    )


def struct(cls: type) -> type:
    """A configuration record: a frozen dataclass whose `Const` fields are folded into the kernel at capture."""
    return dataclass(frozen=True)(cls)


def const_fields(config: object) -> dict[str, object]:
    """The `Const` fields of a configuration instance, by name."""
    if not (is_dataclass(config) and not isinstance(config, type)):
        raise TypeError(f"{config!r} is not a @struct configuration")
    hints = {f.name: f.type for f in fields(config)}
    return {name: getattr(config, name) for name, hint in hints.items() if is_const(hint)}


@dataclass(frozen=True)
class Items:
    """Launch one thread per item."""

    count: int


@dataclass(frozen=True)
class Blocks:
    """An explicit grid of blocks (`threads` is a request the tile lowering may refine)."""

    x: int
    y: int = 1
    z: int = 1
    threads: int | None = None


@dataclass(frozen=True)
class Tiles:
    """One block per tile of an output: the last axis runs along x, the one before along y
    (reference src/krn/frontend/geometry.py:26-39)."""

    shape: tuple[int, ...]
    tile: tuple[int, ...]

    @property
    def blocks(self) -> Blocks:
        counts = [-(-extent // size) for extent, size in zip(self.shape, self.tile, strict=True)]
        return Blocks(*reversed(counts))


class _Index:
    x: int
    y: int
    z: int


class block:
    """The block a kernel body runs in: `block.tile(bm, bn)` is its output tile, `block.index()` its grid position."""

    @staticmethod
    def tile(*sizes: int) -> Any:
        return _stub()

    @staticmethod
    def index() -> _Index:
        return _stub()


zeros = arange = where = maximum = minimum = full = _stub


def pipelined(extent: int, tile: int, *, stages: int | None = None, schedule: object = None) -> Any:
    """The tiles of an axis as slices, software-pipelined by the target (`for ks in pipelined(K, bk)`)."""
    return _stub()


class Kernel:
    """A function that runs on the device (reference src/krn/frontend/kernel.py:22-105).

    `k(*args)` launches with the geometry inferred from the body, `k(..., launch=Tiles(...))` overrides it, and
    `k[Config(...)](...)` passes a configuration struct as the first argument.
    """

    def __init__(self, fn: Any) -> None:
        self.fn = fn
        self.name = getattr(fn, "__name__", type(fn).__name__)
        self._config: type | None | bool = False
        self.parameters = tuple(inspect.signature(fn).parameters)
        self.arity = len(self.parameters)

    def configuration(self) -> type | None:
        """The `@struct` class of the first parameter, if the kernel is configured."""
        if self._config is False:
            parameters = tuple(inspect.signature(self.fn).parameters.values())
            first = parameters[0].annotation if parameters else None
            self._config = first if isinstance(first, type) and is_dataclass(first) else None
        return self._config  # type: ignore[return-value]

    def __call__(self, *args: Any, launch: Any = None, **kwargs: Any) -> None:
        from krn_amd.runtime.api import Configured, Device

        launcher = Device.current().launcher(self, launch.blocks if isinstance(launch, Tiles) else launch)
        config = self.configuration()
        if config is not None and len(args) + len(kwargs) == self.arity - 1:
            launcher = Configured(launcher, config())
        return launcher(*args, **kwargs)

    def __getitem__(self, configuration: Any) -> Any:
        from krn_amd.runtime.api import Configured, Device

        config = self.configuration()
        if config is None or not isinstance(configuration, config):
            raise TypeError(f"{self.name}: brackets take a configuration; pass geometry with launch=")
        return Configured(Device.current().launcher(self), configuration)


def kernel(fn: Any) -> Kernel:
    """The one decorator of device code."""
    return Kernel(fn)

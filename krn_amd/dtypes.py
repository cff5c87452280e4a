"""Element types of the tile path and their arithmetic: the same type stays, a Python literal adopts the other side's
type, and any other mix needs an explicit `.to(...)` (krn's strict arithmetic, reference
src/krn/compiler/dtypes.py:166-180).

Host storage follows krn: bf16 tensors are raw `uint16` words and fp8 tensors are `uint8` codes whose element
type says the format (reference README; tests/compiler/test_tensor_cores.py:305-311).
"""

import typing
from dataclasses import dataclass
from enum import Enum

import numpy as np


class Kind(Enum):
    UINT = "uint"
    SINT = "sint"
    FLOAT = "float"
    BOOL = "bool"
    PY_INT = "py_int"
    PY_FLOAT = "py_float"


@dataclass(frozen=True)
class Dtype:
    """`bits` is the total width and `man` the mantissa width of a float."""

    name: str
    kind: Kind
    bits: int = 0
    man: int = 0

    @property
    def is_int(self) -> bool:
        return self.kind in (Kind.UINT, Kind.SINT)

    @property
    def is_float(self) -> bool:
        return self.kind is Kind.FLOAT

    @property
    def is_py(self) -> bool:
        return self.kind in (Kind.PY_INT, Kind.PY_FLOAT)

    @property
    def is_narrow(self) -> bool:
        """An fp8 format: stored as one-byte codes, decoded before arithmetic."""
        return self.is_float and self.bits == 8

    @property
    def itemsize(self) -> int:
        return max(self.bits // 8, 1)

    def __str__(self) -> str:
        return self.name

    def __repr__(self) -> str:
        return self.name


BOOL = Dtype("bool", Kind.BOOL, 8)
I8 = Dtype("i8", Kind.SINT, 8)
I16 = Dtype("i16", Kind.SINT, 16)
I32 = Dtype("i32", Kind.SINT, 32)
I64 = Dtype("i64", Kind.SINT, 64)
U8 = Dtype("u8", Kind.UINT, 8)
U16 = Dtype("u16", Kind.UINT, 16)
U32 = Dtype("u32", Kind.UINT, 32)
U64 = Dtype("u64", Kind.UINT, 64)
F16 = Dtype("f16", Kind.FLOAT, 16, 10)
BF16 = Dtype("bf16", Kind.FLOAT, 16, 7)
F32 = Dtype("f32", Kind.FLOAT, 32, 23)
F64 = Dtype("f64", Kind.FLOAT, 64, 52)
F8E4M3 = Dtype("f8e4m3fn", Kind.FLOAT, 8, 3)
F8E5M2 = Dtype("f8e5m2", Kind.FLOAT, 8, 2)
PY_INT = Dtype("int", Kind.PY_INT)
PY_FLOAT = Dtype("float", Kind.PY_FLOAT)

BY_NAME = {
    d.name: d
    for d in (BOOL, I8, I16, I32, I64, U8, U16, U32, U64, F16, BF16, F32, F64, F8E4M3, F8E5M2)
}
BY_NAME |= {"bool_": BOOL, "f8e4m3": F8E4M3}

# host storage of each element type
NUMPY = {
    BOOL: np.dtype(np.bool_), I8: np.dtype(np.int8), I16: np.dtype(np.int16), I32: np.dtype(np.int32),
    I64: np.dtype(np.int64), U8: np.dtype(np.uint8), U16: np.dtype(np.uint16), U32: np.dtype(np.uint32),
    U64: np.dtype(np.uint64), F16: np.dtype(np.float16), BF16: np.dtype(np.uint16), F32: np.dtype(np.float32),
    F64: np.dtype(np.float64), F8E4M3: np.dtype(np.uint8), F8E5M2: np.dtype(np.uint8),
}  # fmt: skip

# element type of a host array when no explicit type is given
FROM_NUMPY = {
    np.dtype(np.bool_): BOOL, np.dtype(np.int8): I8, np.dtype(np.int16): I16, np.dtype(np.int32): I32,
    np.dtype(np.int64): I64, np.dtype(np.uint8): U8, np.dtype(np.uint16): U16, np.dtype(np.uint32): U32,
    np.dtype(np.uint64): U64, np.dtype(np.float16): F16, np.dtype(np.float32): F32, np.dtype(np.float64): F64,
}  # fmt: skip


def common(a: Dtype, b: Dtype) -> Dtype | None:
    """The type of `a op b` under strict arithmetic, or None when the mix needs an explicit conversion."""
    if a == b:
        return a
    if a.is_py or b.is_py:
        py, other = (a, b) if a.is_py else (b, a)
        if other.is_py:
            return PY_FLOAT if PY_FLOAT in (a, b) else PY_INT
        accepts = other.is_float or (other.is_int and py.kind is Kind.PY_INT)
        return other if accepts else None
    return None


# krn's element types are parametrised classes (reference src/krn/frontend/numerics.py:343-384): `fp[E, M, kind]`
# with literal exponent and mantissa widths, `sint[N]` and `uint[N]`. (family, parameters) -> the type they name.
_STRUCTURAL = {
    ("fp", (11, 52, "ieee")): F64, ("fp", (8, 23, "ieee")): F32, ("fp", (5, 10, "ieee")): F16,
    ("fp", (8, 7, "ieee")): BF16, ("fp", (4, 3, "fn")): F8E4M3, ("fp", (5, 2, "ieee")): F8E5M2,
    ("sint", (8,)): I8, ("sint", (16,)): I16, ("sint", (32,)): I32, ("sint", (64,)): I64,
    ("uint", (8,)): U8, ("uint", (16,)): U16, ("uint", (32,)): U32, ("uint", (64,)): U64,
}  # fmt: skip


def _parameter(arg: object) -> object:
    """A literal width (`L[8]` -> 8) or a format kind class (`ieee` -> "ieee")."""
    literal = typing.get_args(arg)
    if typing.get_origin(arg) is typing.Literal and len(literal) == 1:
        return literal[0]
    return getattr(arg, "__name__", arg)


def of(value: object) -> Dtype:
    """The element type named by a kernel annotation object, a frontend dtype class of this package, or one of
    krn's own parametrised element types (`fp[L[8], L[7], ieee]` is bf16)."""
    if isinstance(value, Dtype):
        return value
    name = getattr(value, "dtype_name", None) or getattr(value, "__name__", None)
    if name in BY_NAME:
        return BY_NAME[name]
    origin = typing.get_origin(value)
    if origin is not None:
        key = (getattr(origin, "__name__", None), tuple(_parameter(a) for a in typing.get_args(value)))
        if key in _STRUCTURAL:
            return _STRUCTURAL[key]
    raise TypeError(f"{value!r} is not an element type")

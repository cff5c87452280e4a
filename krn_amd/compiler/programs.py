"""Canonical tile programs and the positional renaming that compares two captured programs structurally."""

import dataclasses
from functools import cache
from pathlib import Path

from krn_amd.compiler import ir
from krn_amd.dtypes import F16, Dtype

ATTENTION = Path(__file__).with_name("attention_program.py")
SOFTMAX = Path(__file__).with_name("softmax_program.py")
SOFTMAX_PROGRAMS = ("softmax_long_rows", "softmax", "softmax_steps")


@cache
def _attention(items: tuple, dtype: Dtype) -> ir.Kernel:  # captured in f16, as written
    from krn_amd.compiler.capture import capture

    return capture(ATTENTION, "flash_attention", consts={"t": dict(items)})


def attention(values: dict, dtype: Dtype) -> ir.Kernel:
    """The canonical flash-attention program for one configuration, with `dtype` tensors (f16 in the source; the
    `.to(T.f16)` casts of p and of the output follow the tensors when bf16 is asked for)."""
    kernel = _attention(tuple(sorted(values.items())), F16)
    if dtype == F16:
        return kernel
    return _retype(kernel, F16, dtype)


@cache
def _softmax(name: str, items: tuple) -> ir.Kernel:  # captured in f16, as written
    from krn_amd.compiler.capture import capture

    return capture(SOFTMAX, name, consts={"t": dict(items)})


def softmax(name: str, values: dict, dtype: Dtype) -> ir.Kernel:
    """The canonical row-softmax program `name` for one tiling, with `dtype` tensors (f16 in the source; the
    `.to(T.f16)` casts follow the tensors)."""
    kernel = _softmax(name, tuple(sorted(values.items())))
    if dtype == F16:
        return kernel
    return _drop_same_casts(_retype(kernel, F16, dtype))


def _drop_same_casts(node):
    """`node` without casts to the type their operand already has (capture emits none of those)."""
    if isinstance(node, tuple):
        return tuple(_drop_same_casts(x) for x in node)
    if isinstance(node, ir.Cast) and node.operand.dtype == node.dtype:
        return _drop_same_casts(node.operand)
    if dataclasses.is_dataclass(node) and not isinstance(node, type):
        changes = {f.name: _drop_same_casts(getattr(node, f.name)) for f in dataclasses.fields(node)}
        return dataclasses.replace(node, **changes)
    return node


def _retype(node, old: Dtype, new: Dtype):
    """`node` with every `old` element type replaced by `new`."""
    if isinstance(node, Dtype):
        return new if node == old else node
    if isinstance(node, tuple):
        return tuple(_retype(x, old, new) for x in node)
    if dataclasses.is_dataclass(node) and not isinstance(node, type):
        changes = {f.name: _retype(getattr(node, f.name), old, new) for f in dataclasses.fields(node)}
        return dataclasses.replace(node, **changes)
    return node


def canonical_form(kernel: ir.Kernel) -> tuple:
    """The body and parameter types of `kernel` with variables, parameters and tensors renamed by position."""
    names: dict[str, str] = {}
    params = {name: f"p{i}" for i, (name, _) in enumerate(kernel.params)}

    def rename(node):
        if isinstance(node, tuple):
            return tuple(rename(x) for x in node)
        if isinstance(node, ir.Var):
            return ir.Var(node.type, names.setdefault(node.name, f"v{len(names)}"))
        if isinstance(node, ir.Param):
            return ir.Param(node.type, params[node.name])
        if isinstance(node, ir.TensorRef):
            return ir.TensorRef(params[node.name], node.type)
        if dataclasses.is_dataclass(node) and not isinstance(node, type):
            return dataclasses.replace(node, **{f.name: rename(getattr(node, f.name)) for f in dataclasses.fields(node)
                                                if f.init})
        return node

    return rename(kernel.body), tuple(t for _, t in kernel.params)

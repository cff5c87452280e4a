"""Canonical tile programs and the positional renaming that compares two captured programs structurally."""

import dataclasses
from functools import cache
from pathlib import Path

from krn_amd.compiler import ir
from krn_amd.dtypes import F16, Dtype

ATTENTION = Path(__file__).with_name("attention_program.py")


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

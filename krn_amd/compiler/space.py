"""Launch geometry read from a kernel body: one block per `block.tile` tile of the tensors it stores
(reference src/krn/compiler/space.py:118-138 and frontend/geometry.py:26-39)."""

from collections.abc import Sequence

from krn_amd.frontend import Blocks
from krn_amd.compiler.ir import Dim, Kernel


def extent(dim: Dim, params: dict[str, object]) -> int:
    tensor = params[dim.tensor.name]
    return int(tensor.shape[dim.axis])


def geometry(kernel: Kernel, args: Sequence[object]) -> Blocks:
    """The grid the body asks for: ceil(extent / tile) blocks along each `block.tile` axis, 1 elsewhere. Every
    tensor stored with the same tile must agree on that extent."""
    params = dict(zip((name for name, _ in kernel.params), runtime_args(kernel, args)))
    counts = {"x": 1, "y": 1, "z": 1}
    for axis, size, extents in kernel.space:
        values = {extent(d, params) for d in extents}
        if len(values) > 1:
            raise ValueError(f"{kernel.name}: the tensors tiled along {axis} disagree on its extent: {sorted(values)}")
        counts[axis] = -(-values.pop() // size)
    return Blocks(counts["x"], counts["y"], counts["z"])


def runtime_args(kernel: Kernel, args: Sequence[object]) -> list[object]:
    """The arguments that are runtime parameters: configuration structs are folded at capture and dropped here."""
    names = [name for name, _ in kernel.params]
    if len(args) == len(names):
        return list(args)
    if len(args) == len(kernel.signature):
        runtime = set(names)
        return [a for n, a in zip(kernel.signature, args) if n in runtime]
    raise TypeError(f"{kernel.name} takes {len(names)} runtime arguments, got {len(args)}")

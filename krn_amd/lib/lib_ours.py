"""krn's own kernel behind `lib.matmul` (reference src/krn/lib/lib_ours.py:38-75): the `matmul_epilogue` tile
program with the epilogue chosen by constants, launched on the call's stream. It takes every epilogue, SILU
included. On gfx950 f16 and bf16 operands lower to the MFMA GEMM with the bias and activation fused into its
epilogue; f32 operands to the generic lowering.
"""

from krn_amd.dtypes import BF16, F16, F32
from krn_amd.lib.kernels import MatmulTiling, matmul_epilogue
from krn_amd.lib.lib import Candidate, Epilogue, Op, Operands, Origin, Problem
from krn_amd.runtime.api import Stream

FLAGS = {  # which constants an epilogue sets (reference lib_ours.py:38-46)
    Epilogue.NONE: {},
    Epilogue.BIAS: {"bias": True},
    Epilogue.RELU: {"relu": True},
    Epilogue.GELU: {"gelu": True},
    Epilogue.BIAS_RELU: {"bias": True, "relu": True},
    Epilogue.BIAS_GELU: {"bias": True, "gelu": True},
    Epilogue.SILU: {"silu": True},
}
# the tile the program is written for; the GEMM lowering picks its own MFMA tiles for the whole product
TILE = {"bm": 64, "bn": 64, "bk": 32}


class Ours(Candidate):
    name, op, origin = "ours", Op.MATMUL, Origin.OURS

    def refusal(self, problem: Problem, target=None) -> str | None:
        if len(set(problem.dtypes)) != 1 or problem.dtypes[0] not in (F16, BF16, F32):
            names = ", ".join(str(d) for d in problem.dtypes)
            return f"matmul_epilogue takes one F for a, b, bias and out, f16, bf16 or f32; got {names}"
        return None

    def run(self, problem: Problem, operands: Operands, stream: Stream) -> None:
        a, b, out = operands.a, operands.b, operands.out
        bias = operands.bias if operands.bias is not None else _placeholder(a)  # read only with a bias epilogue
        tiling = MatmulTiling(**TILE, **FLAGS[problem.epilogue])
        with stream:
            matmul_epilogue[tiling](a, b, bias, out)


def _placeholder(a):
    return a.device.empty(a.dtype, 1)


CANDIDATE = Ours()

"""krn's library calls on gfx950: `matmul` with its fused epilogues, dispatched over the reference's AMD candidate
order (hipBLASLt, then krn's own tile program)."""

from krn_amd.lib.lib import Declined, Epilogue, NoCandidate, Operands, Problem, choice, matmul

__all__ = ["Declined", "Epilogue", "NoCandidate", "Operands", "Problem", "choice", "matmul"]

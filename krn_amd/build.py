"""Compile the gfx950 kernel library `libkrn_amd.so` from `krn_amd/csrc` with hipcc, in-tree.

The library is the product: every tile contraction, attention and quantized GEMM launch goes through its C ABI
(include/krn_amd.h). Built for gfx950 only, with packed-FP32 instructions switched off and no FP contraction
outside explicit fused multiply-adds.
"""

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
OUTPUT = PACKAGE / "libkrn_amd.so"
ARCH = "gfx950"
FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-pass-failed",
]  # fmt: skip


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise FileNotFoundError("hipcc not found: install ROCm or put /opt/rocm/bin on PATH")
    return found


def sources() -> list[Path]:
    return sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.cpp")])


def build(verbose: bool = False) -> Path:
    """Compile every source to an object (in parallel), then link the shared library. Always recompiles."""
    objects_dir = PACKAGE / "_build"
    objects_dir.mkdir(exist_ok=True)
    jobs = []
    for source in sources():
        obj = objects_dir / (source.name + ".o")
        command = [hipcc(), *FLAGS, "-I", str(CSRC), "-c", str(source), "-o", str(obj)]
        jobs.append((command, obj, subprocess.Popen(command, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for command, obj, process in jobs:
        output, _ = process.communicate()
        text = "\n".join(
            line for line in output.decode(errors="replace").splitlines() if "packed-fp32-ops" not in line
        )
        if process.returncode:
            failed.append(f"{' '.join(command)}\n{text}")
        elif verbose and text.strip():
            print(text, file=sys.stderr)
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n\n".join(failed))
    temporary = OUTPUT.with_suffix(f".so.{os.getpid()}")
    link = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *(str(o) for _, o, _ in jobs), "-o", str(temporary)]
    result = subprocess.run(link, capture_output=True, text=True)
    if result.returncode:
        raise RuntimeError(f"link failed: {' '.join(link)}\n{result.stdout}{result.stderr}")
    temporary.replace(OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose=True))

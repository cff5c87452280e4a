"""The C ABI on the CPU: `libkrn_amd.so` loads and exports every function `include/krn_amd.h` declares (no compute
call: this container has no GPU)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "krn_amd.h"
LIBRARY = ROOT / "krn_amd" / "libkrn_amd.so"


def declared() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(krn_\w+)\s*\(", text, flags=re.M)


def test_the_header_declares_the_entry_points():
    names = declared()
    assert {"krn_gemm_nt", "krn_attention_fwd", "krn_transpose16", "krn_amd_last_error"} <= set(names)
    assert len(names) == len(set(names))


@pytest.mark.skipif(not LIBRARY.exists(), reason="libkrn_amd.so is not built (run __graft_entry__.build())")
def test_the_library_loads_and_exports_every_declared_function():
    library = ctypes.CDLL(str(LIBRARY))
    missing = [name for name in declared() if not hasattr(library, name)]
    assert not missing, f"declared in include/krn_amd.h but not exported: {missing}"

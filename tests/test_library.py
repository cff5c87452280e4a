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


@pytest.mark.skipif(not LIBRARY.exists(), reason="libkrn_amd.so is not built (run __graft_entry__.build())")
def test_nn_workspace_query_is_zero_exactly_for_the_products_read_as_they_lie():
    """krn_gemm_nn_workspace_for is host arithmetic (no GPU call): 0 for the shapes the kernel reads B K x N as it
    lies (N % 256 == 0, K % 64 == 0, K >= 128, at least 128 tiles of 256 x 256, 16-byte aligned operands),
    otherwise the transposed operand's n * k * 2 bytes."""
    library = ctypes.CDLL(str(LIBRARY))
    query = library.krn_gemm_nn_workspace_for
    query.restype = ctypes.c_int64
    query.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]
    a, b = 1 << 20, 1 << 24  # aligned stand-in addresses: nothing is dereferenced
    assert query(a, b, 8192, 8192, 8192) == 0
    assert query(a, b, 2000, 4096, 192) == 0  # ragged M, an odd number of 128-byte slices
    assert query(a, b, 8192, 8192 + 128, 8192) == (8192 + 128) * 8192 * 2  # N not a multiple of 256
    assert query(a, b, 8192, 8192, 8192 + 32) == 8192 * (8192 + 32) * 2  # K not a multiple of 64
    assert query(a, b, 8192, 8192, 64) == 8192 * 64 * 2  # a single slice
    assert query(a, b, 1024, 4096, 4096) == 4096 * 4096 * 2  # 64 tiles: too few for the whole-tile loop
    assert query(a + 8, b, 8192, 8192, 8192) == 8192 * 8192 * 2  # A not 16-byte aligned
    assert query(a, b + 2, 8192, 8192, 8192) == 8192 * 8192 * 2  # B not 16-byte aligned


@pytest.mark.skipif(not LIBRARY.exists(), reason="libkrn_amd.so is not built (run __graft_entry__.build())")
def test_attention_refuses_what_it_cannot_address_before_any_device_call():
    """krn_attention_fwd checks its arguments on the host and returns -1 with a message before it touches the
    device: an unknown element kind, a head dimension other than 64 or 128, misaligned tensors, no keys, and heads
    whose keys (sk * d * 2 bytes) or whose queries rounded up to a whole 256-row tile ((sq + 256) * d * 2 bytes)
    exceed the 31-bit offsets of its buffer resources."""
    library = ctypes.CDLL(str(LIBRARY))
    fwd = library.krn_attention_fwd
    fwd.restype = ctypes.c_int
    fwd.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                    ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
    library.krn_amd_last_error.restype = ctypes.c_char_p
    p = 1 << 20  # an aligned stand-in address: nothing is dereferenced
    bf16, f32 = 2, 0

    def refused(*args) -> str:
        assert fwd(*args) == -1
        return library.krn_amd_last_error().decode()

    assert "bf16 or f16" in refused(f32, p, p, p, p, 1, 256, 256, 128, 0.1, 1, None)
    assert "head dimension" in refused(bf16, p, p, p, p, 1, 256, 256, 96, 0.1, 1, None)
    assert "aligned" in refused(bf16, p + 2, p, p, p, 1, 256, 256, 128, 0.1, 1, None)
    assert "empty key" in refused(bf16, p, p, p, p, 1, 256, 0, 128, 0.1, 1, None)
    assert "keys" in refused(bf16, p, p, p, p, 1, 256, 1 << 23, 128, 0.1, 1, None)
    assert "queries" in refused(bf16, p, p, p, p, 1, (1 << 23) - 256, 256, 128, 0.1, 1, None)

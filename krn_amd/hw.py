"""Native library loader: the HIP runtime, hiprtc and this package's own gfx950 kernel library.

Mirrors `krn.hw.Libraries` (reference src/krn/hw/libraries.py:324-377): `load(name)` returns a frozen record with the
path and the ctypes handle, `find(name)` only locates, `available(name)` checks loading, and a failure raises
`LibraryNotFound` naming where it looked. The reference has a `"hip"` spec (libraries.py:85-90) and no hiprtc spec;
this module adds `"hiprtc"`, `"hipblaslt"` (the vendor GEMM behind `lib.matmul`'s first AMD candidate, reference
src/krn/lib/lib.py:264 and 516), `"krn_amd"` (the in-tree `libkrn_amd.so`) and `"roctx"` (the reference's ROCTx loader,
src/krn/profile/providers/amd/tracer.py:13-28).
"""

import ctypes
import os
from dataclasses import dataclass
from functools import cache
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent

FILENAMES = {
    "hip": ("libamdhip64.so", "libamdhip64.so.7"),
    "hiprtc": ("libhiprtc.so", "libhiprtc.so.7"),
    "krn_amd": ("libkrn_amd.so",),
    "hipblaslt": ("libhipblaslt.so", "libhipblaslt.so.1"),
    # rocprofv3 (rocprofiler-sdk) records ranges from its own ROCTx library; the older roctracer one is the fallback
    "roctx": ("librocprofiler-sdk-roctx.so", "librocprofiler-sdk-roctx.so.1", "libroctx64.so", "libroctx64.so.4"),
}
FIXES = {
    "hip": "Install ROCm (libamdhip64.so under /opt/rocm/lib)",
    "hiprtc": "Install ROCm (libhiprtc.so under /opt/rocm/lib)",
    "hipblaslt": "Install ROCm's hipBLASLt (libhipblaslt.so under /opt/rocm/lib)",
    "krn_amd": "Build the gfx950 kernels first: python -c 'import __graft_entry__ as g; g.build()'",
    "roctx": "Install ROCm's ROCTx library (librocprofiler-sdk-roctx.so under /opt/rocm/lib)",
}


class LibraryNotFound(OSError):
    """A native library that is not on this machine, with the places searched and how to get it."""

    def __init__(self, name: str, searched: tuple[Path, ...], reason: str = "") -> None:
        self.name, self.searched = name, searched
        where = ", ".join(map(str, searched)) or "nowhere"
        super().__init__(f"{name}: not found ({reason or 'no candidate file'}); searched {where}. {FIXES[name]}")


@dataclass(frozen=True)
class LoadedLibrary:
    name: str
    path: Path
    handle: ctypes.CDLL


def directories(name: str) -> tuple[Path, ...]:
    if name == "krn_amd":
        return (PACKAGE,)
    roots = [Path(os.environ[key]) for key in ("ROCM_PATH", "HIP_PATH") if os.environ.get(key)]
    roots += sorted(Path("/opt").glob("rocm*"))
    return tuple(root / "lib" for root in roots) + (Path("/usr/lib"), Path("/usr/lib/x86_64-linux-gnu"))


class Libraries:
    """Find and load the native libraries the AMD path needs. Loads are cached until `clear_cache()`."""

    @staticmethod
    def find(name: str) -> Path | None:
        for directory in directories(name):
            for filename in FILENAMES[name]:
                if (candidate := directory / filename).exists():
                    return candidate
        return None

    @staticmethod
    @cache
    def load(name: str) -> LoadedLibrary:
        if name not in FILENAMES:
            raise KeyError(f"unknown library {name!r}; known: {', '.join(FILENAMES)}")
        path = Libraries.find(name)
        if path is None:
            raise LibraryNotFound(name, directories(name))
        try:
            handle = ctypes.CDLL(str(path), mode=ctypes.RTLD_GLOBAL)
        except OSError as error:
            raise LibraryNotFound(name, (path,), str(error)) from error
        return LoadedLibrary(name, path, handle)

    @staticmethod
    def available(name: str) -> bool:
        try:
            Libraries.load(name)
        except LibraryNotFound:
            return False
        return True

    @staticmethod
    def clear_cache() -> None:
        Libraries.load.cache_clear()

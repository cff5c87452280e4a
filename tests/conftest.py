import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

KERNELS = ROOT / "tests" / "kernels" / "tile_programs.py"
os.environ.setdefault("KRN_TARGET", "gfx950")


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libkrn_amd.so")


@pytest.fixture(scope="session")
def device():
    """The gfx950 device. The kernel library must be built: a GPU test never falls back to anything else."""
    from krn_amd.runtime.api import device_of

    return device_of("gfx950")

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
if str(ROOT / "tests") not in sys.path:
    sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running CPU case")


def pytest_sessionstart(session):
    """Build the HIP library and the C oracle in-tree if they are missing
    (hipcc cross-compiles for gfx950 without a GPU)."""
    import subprocess
    if not (ROOT / "runnel_amd" / "librmoe.so").exists():
        subprocess.run(["make", "-s", "-j8", "-C", str(ROOT / "runnel_amd" / "csrc")], check=True)
    if not (ROOT / "oracle" / "_build" / "libmoe_oracle.so").exists():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)

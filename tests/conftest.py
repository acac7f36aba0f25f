"""pytest configuration: the `gpu` marker and import paths.

`-m "not gpu"` runs the CPU suite (oracle pins, host logic, library exports);
`-m gpu` runs the parity tests that call libffnerf_hip.so on an MI355X.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "ffnerf-experimental_amd"
for p in (str(ROOT), str(PKG), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def ora():
    from oracle import oracle as o
    o.lib()
    return o

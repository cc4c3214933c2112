"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on CPU."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


@pytest.fixture(scope="session")
def ora():
    """The CPU oracle (built on demand; test infrastructure only)."""
    from oracle import ora as _ora
    _ora.lib()
    return _ora


@pytest.fixture(scope="session")
def rai():
    import rai_amd
    rai_amd.lib()
    return rai_amd


def golden(name: str) -> str:
    return os.path.join(GOLDEN, name)


def read_golden(name: str) -> bytes:
    with open(golden(name), "rb") as f:
        return f.read()

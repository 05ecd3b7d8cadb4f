"""Shared test setup.

Markers: `gpu` tests need a real MI355X and call the HIP library through the
C ABI; everything else runs on the CPU.  The oracle (oracle/) is the checker
in both.
"""
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT / "volta-zk_amd", ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running (full-size) case")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.build()
    return o


@pytest.fixture(scope="session")
def backend():
    """One resident context for the GPU session.  Fails (never skips) when the
    library or the GPU is missing: GPU tests must exercise the HIP path."""
    from volta_mi355x import Backend
    b = Backend()
    yield b
    b.close()

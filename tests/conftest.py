"""Shared pytest setup: markers, import paths, oracle and GPU fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gemma4.kt_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libg4hip.so on cuda:0)")


@pytest.fixture(scope="session")
def oracle():
    import oracle as _oracle
    _oracle.lib()
    return _oracle


@pytest.fixture(scope="session")
def g4():
    import g4hip
    g4hip.lib()
    return g4hip


@pytest.fixture(scope="session")
def ctx(g4):
    """One library context on device 0 for the whole GPU session."""
    if g4.device_count() == 0:
        pytest.fail("GPU test selected but no HIP device is visible")
    c = g4.Context(0)
    yield c
    c.close()


def announce(msg: str) -> None:
    """Name the case before a GPU step (flushed, so it survives a lost box)."""
    print("[case] " + msg, flush=True)

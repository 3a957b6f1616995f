"""Shared fixtures. `gpu`-marked tests need a real MI355X; everything else runs on the CPU."""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("rocket-userspace_amd", "oracle"):
    p = os.path.join(REPO, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through librocketnpu's C-ABI)")


@pytest.fixture(scope="session")
def lib():
    import rocketnpu
    return rocketnpu.load()


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def fd(lib):
    """An open handle on cuda:0. A GPU test that cannot open one fails: no fallback."""
    h = lib.rocket_open()
    assert h >= 0, f"rocket_open() = {h}: no MI355X visible"
    yield h
    lib.rocket_close(h)

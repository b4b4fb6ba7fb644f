import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libzkie_hip.so)")
    config.addinivalue_line("markers", "slow: full-size configuration")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    O.lib()
    return O


@pytest.fixture(scope="session")
def emu():
    """Host build of the device code (tests/emu/emu.cpp)."""
    from tests.emu import emu as E

    return E.load()


@pytest.fixture(scope="session")
def native():
    """The HIP library; GPU tests fail loudly if it is missing."""
    from zkie_amd import _native as N

    lib = N.load()
    assert N.device_count() > 0, "no HIP device visible"
    return N

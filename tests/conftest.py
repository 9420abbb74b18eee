import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libsoso_hip.so on the device)")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gpu():
    """One HipGpu handle for the whole GPU session (one process on the card)."""
    from soso_amd.dispatch import HipGpu
    g = HipGpu(0)
    yield g
    g.close()

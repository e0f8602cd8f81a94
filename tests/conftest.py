import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def orc():
    import oracle

    if not os.path.exists(oracle._LIB_PATH):
        oracle.build()
    return oracle


@pytest.fixture(scope="session")
def hip():
    """The C ABI, initialised on device 0. GPU tests only."""
    from neuralrs_amd import _abi

    _abi.load()
    _abi.init(0)
    return _abi

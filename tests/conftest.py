import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs on the MI355X box)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def oracle():
    """The CPU oracle (test infrastructure); built from oracle/ if missing."""
    import oracle as O

    O.build()
    O.lib()
    return O


@pytest.fixture(scope="session")
def gpu():
    """libnrq initialised on device 0; fails loudly if it cannot be."""
    import torch

    import nightrun_amd
    from nightrun_amd import _lib

    assert torch.cuda.is_available(), "GPU test needs a visible gfx950 device"
    _lib.lib()
    nightrun_amd.init(0)
    return nightrun_amd

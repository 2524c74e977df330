import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and libssa_hip.so")


@pytest.fixture(scope="session")
def dev():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible AMD GPU"
    import ssa_amd

    ssa_amd._lib.load()
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle

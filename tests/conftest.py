import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libxtag_eva.so")
    config.addinivalue_line("markers", "slow: long-running (minutes)")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def xt():
    from xtagger_amd import lib as L
    return L


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as O
    return O

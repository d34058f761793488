"""Shared pytest setup: the `gpu` marker, the package and oracle handles."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


@pytest.fixture(scope="session")
def sqa():
    import __graft_entry__ as ge

    return ge.load_package()


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o

    if not os.path.exists(o.LIB_PATH):
        o.build()
    return o


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")

import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950)")


@pytest.fixture(scope="session")
def lib():
    import tqt_testlib

    return tqt_testlib.load_product_module().load()


@pytest.fixture(scope="session")
def shim():
    import ctypes

    import tqt_testlib

    if not os.path.exists(tqt_testlib.SHIM_SO):
        pytest.fail("test shim not built: %s" % tqt_testlib.SHIM_SO)
    return ctypes.CDLL(tqt_testlib.SHIM_SO)


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test requested but torch.cuda.is_available() is False")
    return torch.device("cuda:0")

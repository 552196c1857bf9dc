import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libcpq.so")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    O.lib()  # builds the oracle once if its shared object is missing
    return O


@pytest.fixture(scope="session")
def device():
    """The HIP device; GPU tests fail loudly (never skip) when it is absent."""
    from cider_press_amd.kernels import Device

    return Device.system_default()


@pytest.fixture(scope="session")
def library(device):
    from cider_press_amd.kernels import KernelLibrary

    return KernelLibrary.quantized(device)

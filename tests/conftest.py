import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (gfx950); runs through libcbxops' C ABI")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    O.lib()
    return O


@pytest.fixture(scope="session")
def cbx():
    import torch

    from chatterbox_amdvulkan_amd import cbxops

    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    cbxops.load()
    cbxops.init(0)
    return cbxops

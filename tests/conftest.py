import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (runs through librustral_kv.so on cuda:0)")


@pytest.fixture(scope="session")
def dev():
    import torch
    assert torch.cuda.is_available(), "gpu-marked test run without a visible GPU"
    from rustral_amd import _lib
    _lib.lib()  # loud failure if the HIP library is missing
    return torch.device("cuda:0")

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libbrain_hip.so on cuda:0)")


@pytest.fixture(scope="session")
def gpu():
    """The GPU tests' device. Fails (never skips) without a GPU: a GPU test
    that silently did nothing would hide a broken native path."""
    import torch

    assert torch.cuda.is_available(), "gpu-marked test needs a HIP device"
    import brain_amd

    brain_amd.load()
    return torch.device("cuda:0")

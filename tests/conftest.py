import os
import sys

import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (os.path.join(REPO, "kalman-linear-attention_amd"), REPO):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) GPU and the built libkla_hip.so")
    config.addinivalue_line("markers", "slow: long-running CPU check (gradcheck and the like)")


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(0)


@pytest.fixture
def cuda():
    """The GPU tests' device; fails (does not skip) without a GPU."""
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return torch.device("cuda", 0)

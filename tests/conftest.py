import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built library")


@pytest.fixture
def gpu():
    """Device fixture for GPU tests: fails (never skips) when no GPU is visible."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return torch.device("cuda:0")

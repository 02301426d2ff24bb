import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; fails (does not skip) when none is visible, so a GPU
    run without a GPU cannot pass silently."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return torch.device("cuda:0")

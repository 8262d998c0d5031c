import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "kriya-rt_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def kq():
    """The product binding; a GPU test fails (never skips) when the GPU or the library is missing."""
    import torch

    import kriya_q4

    assert torch.cuda.is_available(), "GPU test run without a GPU"
    kriya_q4.lib()
    return kriya_q4

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "tests"), os.path.join(ROOT, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (runs the HIP library on cuda:0)")


@pytest.fixture(scope="session")
def gpu():
    """The GPU tests run where a GPU is: fail, never skip, without one."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    torch.cuda.init()
    return torch.device("cuda:0")

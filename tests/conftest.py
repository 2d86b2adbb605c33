import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

GOLDEN = os.path.join(REPO, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def cuda():
    """The GPU device; GPU tests fail (not skip) when there is none, so a
    silent CPU run can never pass for a GPU parity run."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return torch.device("cuda:0")

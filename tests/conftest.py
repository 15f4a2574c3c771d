import os
import sys
from pathlib import Path

import pytest

REPO_ROOT = Path(__file__).resolve().parent.parent
if str(REPO_ROOT) not in sys.path:
    sys.path.insert(0, str(REPO_ROOT))


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs a HIP device (MI355X / gfx950) and the built library")


@pytest.fixture(scope="session")
def hip_device():
    """cuda:0 for GPU tests; skips only when the host has no HIP device."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device on this host")
    return torch.device("cuda:0")

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; GPU tests fail (not skip) without one, since they only
    run when selected with ``-m gpu`` on a GPU machine."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    from awesome_acceleration_amd import _lib
    _lib.lib()  # fail loudly if the extension is missing
    return torch.device("cuda:0")

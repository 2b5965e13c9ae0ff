import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu():
    """The HIP path: torch device + loaded libds4hip.so. Fails (not skips)
    when the library is missing, so a GPU run never passes on a fallback."""
    import torch
    from ds4cuda_amd import lib
    assert torch.cuda.is_available(), "gpu tests need a GPU"
    lib()
    return torch.device("cuda:0")

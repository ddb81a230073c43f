import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; GPU tests fail (they do not skip) when none is visible, since they are only selected where
    one is expected."""
    import torch

    assert torch.cuda.is_available(), "no GPU visible: run the gpu-marked tests on an MI355X"
    return torch.device("cuda", 0)

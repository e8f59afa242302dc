import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; fails loudly (no silent skip) when a gpu-marked test runs without the built library."""
    import torch

    from karpo_decision_amd import _lib

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    _lib.load()  # raises when the library is missing: never a fallback
    return torch.device("cuda", 0)

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs on the GPU box")
    config.addinivalue_line("markers", "slow: longer CPU-side oracle runs")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    if not oracle.LIB_PATH.exists():
        oracle.build()
    return oracle


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Device fixture for GPU tests: fails (not skips) when no GPU is visible,
    so a GPU run never passes silently on a CPU host."""
    if not _gpu_available():
        pytest.fail("GPU test selected but torch sees no HIP device")
    import torch

    return torch.device("cuda:0")

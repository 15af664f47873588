import sys
import zlib
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built kernel library")


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with the kernel library loaded. Skips without a GPU; raises (fails) if the library is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from foidfinder_amd import kernels

    kernels.lib()
    return torch.device("cuda:0")


@pytest.fixture
def rng(request):
    """Seeded per test (from its name) so every case is reproducible and named in the log."""
    return np.random.default_rng(zlib.crc32(request.node.name.encode()))

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running case")


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle


@pytest.fixture(scope="session")
def hip_ready():
    """Loads the kernel library and selects device 0 (GPU tests only)."""
    import cactus_amd
    n = cactus_amd.device_count()
    assert n >= 1, "GPU tests need a visible GPU"
    cactus_amd.call("cactus_hip_init", 0)
    return cactus_amd

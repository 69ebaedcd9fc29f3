import os
import random
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

REPO = Path(__file__).resolve().parent.parent
for p in (REPO / "tt-cadlab_amd", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(autouse=True)
def reset_seeds():
    # the reference's test seed (tests/conftest.py:10-15)
    torch.manual_seed(213919)
    np.random.seed(213919)
    random.seed(213919)
    torch.set_num_threads(min(8, os.cpu_count() or 1))


@pytest.fixture(scope="session")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from palu_tt import _native
    _native.load()  # the HIP library must be there: a missing build fails the test, never falls back
    return torch.device("cuda:0")

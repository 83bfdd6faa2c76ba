import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X, gfx950)")


def golden(name: str):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def dev():
    """The HIP device for GPU tests; the native library must be the code that runs."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import forge_amd
    forge_amd.load()   # raises if libforge_amd.so is missing: no fallback path exists
    return torch.device("cuda:0")

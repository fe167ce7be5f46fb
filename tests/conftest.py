import importlib
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden", "sampling_golden.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built libgse.so")


@pytest.fixture(scope="session")
def ge():
    return importlib.import_module("goethe-engine_amd")


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def gpu(ge):
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test without a HIP device")
    return torch.device("cuda", 0)

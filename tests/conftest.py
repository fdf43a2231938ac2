import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.dirname(os.path.abspath(__file__))
for p in (REPO, TESTS):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def ora():
    from oracle import pyoracle

    pyoracle.lib()
    return pyoracle


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    return np.load(os.path.join(TESTS, "golden", "dequant_ref.npz"), allow_pickle=False)


@pytest.fixture(scope="session")
def gpu():
    """The HIP operator library on cuda:0. Fails (never skips) when the library
    or the device is missing, so a GPU run cannot pass on a fallback."""
    import torch

    from rpgbarenginecuda_amd import ops

    assert torch.cuda.is_available(), "GPU tests need a visible device"
    ops.load_library()
    ops.init()
    ok, desc = ops.device_info()
    assert ok, desc
    print(f"\n[gpu] {desc}", flush=True)
    return ops

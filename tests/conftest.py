import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libvoxhip.so")
    config.addinivalue_line("markers", "ref: needs oracle/_ref (the compiled reference harness)")


@pytest.fixture(scope="session")
def oracle():
    import pyoracle
    pyoracle.lib()
    return pyoracle


@pytest.fixture(scope="session")
def ref(oracle):
    if oracle.ref() is None:
        pytest.skip("oracle/_ref is not built (the reference sources are not present here)")
    return oracle


@pytest.fixture(scope="session")
def hip():
    """The product library on cuda:0 equivalent (HIP device 0). No fallback: fails when absent."""
    from vox_amd import voxhip
    voxhip.init("hip:0")
    return voxhip


def rel_err(a, b):
    """The reference's `vox verify` metric: max|a - b| / max(1, max|b|) (cli/main.cpp:796-803)."""
    import numpy as np
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(1.0, float(np.max(np.abs(b)))))

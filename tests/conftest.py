import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running CPU oracle case")


def pytest_collection_modifyitems(config, items):
    # GPU tests must run where a GPU exists; say so instead of failing obscurely.
    pass


@pytest.fixture(scope="session")
def oracle():
    from oracle import pyoracle
    pyoracle.lib()
    return pyoracle


@pytest.fixture(scope="session")
def hip():
    """The HIP library (raises when it is not built: there is no CPU fallback)."""
    from mlxcat_amd import _lib
    L = _lib.load()
    rc = L.mc_set_device(0)
    if rc < 0:
        raise RuntimeError(L.mc_last_error().decode())
    return _lib

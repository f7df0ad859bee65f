import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "retrieval-is-not-always-needed_amd")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def load_pkg():
    """Import the product package (its directory name is not an identifier)."""
    if "rina_amd" in sys.modules:
        return sys.modules["rina_amd"]
    spec = importlib.util.spec_from_file_location("rina_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["rina_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device; calls through the HIP C-ABI")
    config.addinivalue_line("markers", "slow: full-size shapes")


@pytest.fixture(autouse=True)
def _release_device_tensors():
    yield
    import _util
    if _util.LIVE:
        _util.torch().cuda.synchronize()
        _util.LIVE.clear()


@pytest.fixture(scope="session")
def rina():
    return load_pkg()


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.load()
    return oracle

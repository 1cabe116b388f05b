import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP kernel library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def reference():
    from oracle import Reference
    if not Reference.available():
        pytest.skip("reference CPU path not built (needs the reference sources: make -C oracle ref)")
    return Reference()


@pytest.fixture()
def compute():
    """A ROCm provider context on the real HIP runtime; creation failure is
    a test failure, never a skip."""
    from fyodor_amd import Compute
    os.environ.pop("NYA_ROCM_HIP_LIBRARY", None)
    os.environ.pop("NYA_ROCM_CACHE_MIB", None)
    c = Compute("rocm")
    assert c.name == "rocm"
    yield c
    c.close()

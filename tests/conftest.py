import os
import subprocess
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


@pytest.fixture(scope="session")
def mock_paths(tmp_path_factory):
    """The mock HIP runtime + kernel library (tests/mock/mock_hip.c), and a
    copy of it without hipInit (a library missing a symbol)."""
    out = tmp_path_factory.mktemp("mock")
    src = [str(REPO / "tests/mock/mock_hip.c"), str(REPO / "oracle/quant_oracle.c")]
    good, missing = out / "libnya_mock_hip.so", out / "libnya_mock_missing.so"
    base = ["gcc", "-std=c17", "-O1", "-fPIC", "-shared", "-D_POSIX_C_SOURCE=200809L"]
    subprocess.run(base + src + ["-o", str(good), "-lm", "-lpthread"], check=True)
    subprocess.run(base + ["-DhipInit=nya_mock_unused_init"] + src + ["-o", str(missing), "-lm", "-lpthread"], check=True)
    return good, missing


DROPIN_LIBRARY = REPO / "oracle" / "_ref" / "libnya_dropin.so"


@pytest.fixture(scope="session")
def dropin_library():
    """The engine's own dispatcher, CPU provider and caller
    (backend/core/compute.c, cpu_backend.c, llm_quant.c, vendor.c) built
    from the reference sources with this repository's rocm.c registered
    (make -C oracle dropin); skipped where the reference sources are not
    mounted."""
    import ctypes
    from fyodor_amd import compute_api
    proc = subprocess.run(["make", "-C", str(REPO / "oracle"), "dropin"], capture_output=True, text=True)
    if proc.returncode != 0 or not DROPIN_LIBRARY.exists():
        pytest.skip("reference sources not mounted: the drop-in build needs backend/core from the reference tree")
    return compute_api(ctypes.CDLL(str(DROPIN_LIBRARY)))

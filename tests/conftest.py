"""Shared test setup: import paths, the `gpu` marker and oracle/HIP builds."""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "sx8-quantization_amd")
ORACLE = os.path.join(REPO, "oracle")
for p in (REPO, PKG, ORACLE):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (run with -m gpu)")


@pytest.fixture(scope="session")
def oracle():
    import oracle as O
    if not os.path.exists(O.LIB_PATH):
        O.build()
    O.lib()
    return O


@pytest.fixture(scope="session")
def hiplib():
    """The built HIP library (built on demand on the CPU side; on the GPU box it is
    shipped prebuilt and only loaded)."""
    import _sx8lib
    if not os.path.exists(_sx8lib.lib_path()):
        _sx8lib.build()
    return _sx8lib.lib()


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


@pytest.fixture
def gemm_tuning(hiplib):
    """Setter for the prefill tuning variables (TILE=, PLAN=, W2=) during one test; the
    library reads them once, so the setter and the teardown make it read them again."""
    import _sx8lib
    t = _sx8lib.GemmTuning()
    yield t.set
    t.restore()

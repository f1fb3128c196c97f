import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle import Ref
    return Ref()


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _library_defaults(request):
    """Every GPU test starts from the library's default switches: the
    process-wide activation mode (set by the dual op's callers) and the
    tuning keys a test may change are put back after it."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    import llapis_amd as la
    lib = la.lib()
    lib.llapis_set_modes(la.ACT_CPU, la.GELU_TABLE)
    for key, value in ((0, 1), (2, 1), (3, -1), (4, -1), (6, 1)):
        lib.llapis_set_tuning(key, value)

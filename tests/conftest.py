import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm GPU) and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def gpu_ready() -> bool:
    import torch

    return torch.cuda.is_available() and getattr(torch.version, "hip", None) is not None


@pytest.fixture
def dev():
    import torch

    if not gpu_ready():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _require_hip_for_gpu_tests(request, monkeypatch):
    """GPU tests run with TRNBLAS_REQUIRE_HIP semantics: a kernel error
    raises instead of falling back to torch, so a pass means the HIP path ran."""
    if request.node.get_closest_marker("gpu") is not None:
        from trnblas_amd.hip import dispatch

        monkeypatch.setattr(dispatch, "_REQUIRE_HIP", True)

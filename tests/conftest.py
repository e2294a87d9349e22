import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a GPU; run with -m 'not gpu'")
    return torch.device("cuda:0")


@pytest.fixture
def plan():
    """Pin launch-plan knobs for one test: plan("OC_GEMM_MT", 2).  Cleared afterwards."""
    from onecompression_amd import _native as N

    yield N.set_plan_override
    N.clear_plan_overrides()

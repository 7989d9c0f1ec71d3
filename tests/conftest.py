import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO, "starrygl-unidyngraph_amd")
for p in (REPO, PKG_ROOT, os.path.join(REPO, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(REPO, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI library)")
    # the CPU oracle on one thread: torch's multithreaded fp32 CPU kernels
    # round differently from process to process, and the teacher-forced tests
    # follow the oracle's own parameter trajectory, so its steps must be
    # reproducible for the comparisons to be
    import torch
    torch.set_num_threads(1)


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Device handle for GPU tests; fails (never silently skips) when no GPU."""
    import torch
    if not _gpu_available():
        pytest.fail("GPU test collected without a GPU (run with -m 'not gpu' on CPU hosts)")
    return torch.device("cuda:0")

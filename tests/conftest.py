import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def _has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def qm():
    """The product package (its directory name is not an identifier)."""
    import __graft_entry__
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def gpu(qm):
    """Skip unless a GPU is present; then the native library must load."""
    if not _has_gpu():
        pytest.skip("no GPU in this environment")
    qm.native.load()  # raises if the HIP library is missing: no silent fallback
    return qm

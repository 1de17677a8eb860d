import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)
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


def pytest_terminal_summary(terminalreporter):
    """The achieved parity margins (tests/margins.py), one line per test and kind."""
    from margins import summary
    rows = summary()
    if not rows:
        return
    terminalreporter.section("parity margins (worst per test; bar where the test names it)")
    for test, kind, v, bar in rows:
        tail = f"  bar {bar:g}  ({v / bar:.1%} of it)" if isinstance(bar, (int, float)) and bar > 0 else ""
        terminalreporter.write_line(f"{kind:>4} {v:.3e}{tail}  {test}")

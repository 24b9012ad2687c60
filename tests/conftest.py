import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libqwen_gpu.so's C ABI)")


@pytest.fixture(scope="session")
def qgl():
    """libqwen_gpu.so bound (GPU tests only)."""
    from nebula_amd import qg
    return qg.lib()

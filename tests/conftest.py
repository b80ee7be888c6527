import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "atomic_ai_hybrid-v0.1_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def lib():
    """The built C-ABI library (``libatomic_hybrid.so``).  GPU tests fail
    loudly when it is missing rather than falling back to anything."""
    from atomic_ops import _lib
    return _lib.load()

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def gpu_ctx():
    """One library context on device 0 for the whole GPU session (one process, one context)."""
    from vesper_amd import _lib
    lib = _lib.load()
    if lib.device_count() < 1:
        pytest.skip("no HIP device visible")
    ctx = _lib.Context(0)
    yield ctx
    ctx.close()

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


def _supports_direct_io(directory: Path) -> bool:
    probe = directory / ".direct_probe"
    try:
        probe.write_bytes(b"\0" * 4096)
        handle = os.open(probe, os.O_RDONLY | os.O_DIRECT)
        os.close(handle)
        return True
    except OSError:
        return False
    finally:
        probe.unlink(missing_ok=True)


@pytest.fixture
def direct_io_dir(tmp_path):
    """A directory whose filesystem accepts O_DIRECT opens (the store reader has no buffered fallback):
    pytest's tmp_path when it does, else a temporary directory beside the repository, removed afterwards."""
    import shutil
    import tempfile
    if _supports_direct_io(tmp_path):
        yield tmp_path
        return
    directory = Path(tempfile.mkdtemp(prefix=".direct_io_", dir=ROOT))
    try:
        if not _supports_direct_io(directory):
            pytest.skip("no filesystem here accepts O_DIRECT")
        yield directory
    finally:
        shutil.rmtree(directory, ignore_errors=True)

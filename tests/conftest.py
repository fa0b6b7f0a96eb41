import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libouro_hip.so")


@pytest.fixture(scope="session")
def gpu():
    """Initialise libouro_hip on the GPU; the library must be present."""
    from ouroboros_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} missing: the HIP extension was not built")
    if not _lib.gpu_available():
        pytest.skip("no HIP device visible")
    _lib.init(int(os.environ.get("OURO_GPU_INDEX", "-1")))
    return _lib.lib()


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle

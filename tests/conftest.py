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


# Achieved error margins of the floating-point parity tests, printed at the
# end of the run so a drift toward a bar is visible before it fails.
_MARGINS = []


@pytest.fixture
def margin(request):
    """margin(label, got, want, bar) -> (max|err| / max|want|, L2 ratio).

    Also records the largest elementwise relative error over the entries
    with |want| >= 1 % of max|want| (smaller entries are cancellation noise
    for a normwise bar)."""
    import numpy as np

    def rec(label, got, want, bar):
        g = np.asarray(got, np.float64)
        w = np.asarray(want, np.float64)
        d = np.abs(g - w)
        scale = max(float(np.abs(w).max()), 1e-30)
        norm = float(d.max()) / scale if d.size else 0.0
        l2 = float(np.linalg.norm(d) / max(np.linalg.norm(w), 1e-30))
        big = np.abs(w) >= 1e-2 * scale
        elem = float((d[big] / np.abs(w[big])).max()) if big.any() else 0.0
        _MARGINS.append((request.node.name, label, norm, l2, elem, bar))
        return norm, l2

    return rec


def pytest_terminal_summary(terminalreporter):
    if not _MARGINS:
        return
    tr = terminalreporter
    tr.write_sep("-", "achieved error margins")
    tr.write_line(f"{'test':58} {'tensor':18} {'max/max':>9} {'L2':>9} {'elem>=1%':>9} {'bar':>7}")
    for name, label, norm, l2, elem, bar in _MARGINS:
        tr.write_line(f"{name[:58]:58} {label[:18]:18} {norm:9.2e} {l2:9.2e} {elem:9.2e} {bar:7.0e}")

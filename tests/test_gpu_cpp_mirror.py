"""The reference's own unit tests for this path, restated in C++ against the
C++ host mirror (include/ouro/infer.hpp), run on the GPU."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
BIN = Path(__file__).resolve().parent / "cpp" / "reference_kats"


def test_reference_kats_through_cpp_mirror(gpu):
    if not BIN.exists():
        pytest.fail(f"{BIN} missing: run __graft_entry__.build()")
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("PASS") == 13

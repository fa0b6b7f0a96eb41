"""The C++ host mirror's BMTS reader (include/ouro/bmts.hpp) against the
reference's format tests, compiled and run on the host (no device)."""
import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "cpp" / "bmts_kats.cpp"


def test_bmts_kats_through_cpp_mirror(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no g++")
    exe = tmp_path / "bmts_kats"
    build = subprocess.run([cxx, "-O1", "-std=c++17", "-Wall", "-Werror", str(SRC), "-o", str(exe)],
                           capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    r = subprocess.run([str(exe), str(tmp_path)], capture_output=True, text=True, timeout=60)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("PASS") == 4

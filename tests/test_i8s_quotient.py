"""The GEMM epilogues' reciprocal form of bitnet.cpp's (acc / s) quotient
(i8s_out_inv, ouroboros_amd/csrc/common.hpp) against the IEEE division, for
every integer accumulator |acc| <= 2^20 and a spread of I8_S activation
scales, compiled and run on the host (no device).  The GPU tests then hold
the kernels that use it bit-exact against the oracle's division."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "cpp" / "i8s_quotient_check.c"


def test_reciprocal_quotient_equals_division(tmp_path):
    cc = shutil.which("gcc")
    if cc is None:
        pytest.skip("no gcc")
    exe = tmp_path / "i8s_quotient_check"
    # -ffp-contract=off: the product q = a * inv must round on its own, as on the device
    build = subprocess.run([cc, "-O2", "-ffp-contract=off", "-Wall", "-Werror", str(SRC), "-o", str(exe), "-lm"],
                           capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    r = subprocess.run([str(exe), "400"], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    m = re.search(r"checked (\d+) mismatches (\d+)", r.stdout)
    assert m and r.returncode == 0, r.stdout + r.stderr
    assert int(m.group(1)) > 8e8 and int(m.group(2)) == 0

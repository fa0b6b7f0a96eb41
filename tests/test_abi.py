"""The C-ABI library loads and exports every entry point of include/*.h.
No compute is launched here (no GPU on this tier)."""
import re
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(ouro_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_functions()
    for must in ("ouro_matvec_q", "ouro_matmul_q", "ouro_gemm_i2", "ouro_fwht_rows",
                 "ouro_rotate_fwd", "ouro_rotate_inv", "ouro_delta_head_dim", "ouro_gdn_decode"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from ouroboros_amd import _lib

    lib = _lib.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert set(declared_functions()) <= set(_lib.SIGNATURES), "ctypes binding lags the header"


def test_calls_before_init_fail_cleanly():
    # A fresh process: every entry point refuses with OURO_ERR_NOT_INIT.
    code = (
        "import ctypes as C; from ouroboros_amd import _lib; L=_lib.lib(); "
        "assert L.ouro_matvec_q(None,143,4,128,None,None,None)==7; "
        "assert L.ouro_fwht_rows(None,0,None,0,1,16,16,None,0,None,None,None)==7; "
        "assert b'ouro_init' in L.ouro_last_error(); print('ok')"
    )
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True)
    assert r.returncode == 0 and "ok" in r.stdout, r.stderr


def test_init_without_gpu_reports_no_device():
    from ouroboros_amd import _lib

    if _lib.gpu_available():
        pytest.skip("a GPU is visible here")
    code = ("from ouroboros_amd import _lib; L=_lib.lib(); st=L.ouro_init(-1); "
            "print(st, L.ouro_last_error().decode())")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert r.stdout.split()[0] == "5"  # OURO_ERR_NO_DEVICE, no abort


def test_i2_tiled_bytes_matches_oracle(orc):
    from ouroboros_amd import ops

    for out_len, in_len in ((6912, 2560), (2560, 6912), (13, 256), (5, 1024), (7, 300)):
        want = orc.lib().orc_i2_tiled_bytes(out_len, in_len)
        assert ops.i2_tiled_bytes(out_len, in_len) == want


def test_chunk_workspace_bytes():
    from ouroboros_amd import qwen35

    rec = 9472  # T operands 8.5 KiB (six dense blocks, four diagonal blocks by their 40 non-zero lanes) + beta, g, nk [64] fp32
    assert qwen35.chunk_workspace_bytes(16384, 4, 32) == (256 + 4 + 1) * 32 * rec
    assert qwen35.chunk_workspace_bytes(100, 1000, 2) == (1 + 256 + 1) * 2 * rec
    assert qwen35.chunk_workspace_bytes(64, 1, 4, d=64) == 0
    assert qwen35.chunk_workspace_bytes(64, 1, 4, chunk=32) == 0


def test_no_oracle_in_product():
    # The product never imports, links or loads the oracle.
    for p in list((ROOT / "ouroboros_amd").rglob("*.py")) + list((ROOT / "ouroboros_amd" / "csrc").glob("*")):
        text = p.read_text(errors="ignore")
        assert "import oracle" not in text and "ouro_oracle" not in text and "orc_" not in text, p


def test_layer_workspace_bytes():
    from ouroboros_amd import qwen35

    # the layer block is one launch and keeps nothing between kernels
    assert qwen35.layer_workspace_bytes(32, 16, 32) == 0
    assert qwen35.layer_workspace_bytes(3, 2, 6) == 0
    assert qwen35.layer_workspace_bytes(32, 16, 32, d=64) == 0

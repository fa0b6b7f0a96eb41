"""The committed golden fixtures still come out of the oracle bit for bit
(guards the oracle against drift)."""
from pathlib import Path

import numpy as np

G = Path(__file__).resolve().parent / "golden"


def test_tl1(orc):
    f = np.load(G / "tl1_matvec_37x384.npz")
    n, k = int(f["out_len"]), int(f["in_len"])
    assert np.array_equal(orc.matvec_tl1(f["payload"], n, k, f["x"], simd=0), f["y_scalar"])
    assert np.array_equal(orc.matvec_tl1(f["payload"], n, k, f["x"], simd=1), f["y_sse"])


def test_i2s(orc):
    f = np.load(G / "i2s_gemm_40x512x3.npz")
    xq, s = orc.act_quant_i8(f["x"])
    assert np.array_equal(xq, f["xq"]) and np.array_equal(s, f["act_scale"])
    acc, y = orc.gemm_i2s(f["i2s"], 40, 512, xq, s)
    assert np.array_equal(acc, f["acc"]) and np.array_equal(y, f["y"])
    assert np.array_equal(orc.i2_tile(orc.i2s_to_canonical(f["i2s"], 40, 512), 40, 512), f["tiled"])


def test_hadamard(orc):
    f = np.load(G / "hadamard.npz")
    a = f["fwd_x"].copy()
    orc.rotate_fwd(a, f["fwd_signs"], 16)
    assert np.array_equal(a, f["fwd_y"])
    b = f["inv_x"].copy()
    orc.rotate_inv(b, f["inv_signs"], 16)
    assert np.array_equal(b, f["inv_y"])
    r = (f["rows_x_bf16"].astype(np.uint32) << 16).view(np.float32).copy()
    orc.rotate_rows(r, None, 4096)
    assert np.array_equal(r, f["rows_y_f32"])


def bf(x):
    return (x.astype(np.uint32) << 16).view(np.float32)


def test_gdn(orc):
    f = np.load(G / "gdn_decode_b1.npz")
    s = f["state"].copy()
    o = orc.gdn_decode(s, bf(f["q"]), bf(f["k"]), bf(f["v"]), f["gate"], f["beta"], 1, 1, 2, 128, 3, 1e-6)
    assert np.array_equal(o, f["out"]) and np.array_equal(s, f["state_out"])
    f = np.load(G / "gdn_prefill_t70.npz")
    s = f["state"].copy()
    o = orc.gdn_prefill_tokens(s, bf(f["q"]), bf(f["k"]), bf(f["v"]), f["gate"], f["beta"], 70, 1, 2, 128, 3, 1e-6)
    assert np.array_equal(o, f["out"]) and np.array_equal(s, f["state_out"])

"""Write the golden fixtures of this directory from the CPU oracle.

The reference (Rust) cannot be built or run here, so the expected outputs
come from the oracle (oracle/, pinned by the reference's own KATs).  The
inputs reuse the reference tests' byte patterns where one exists
(ops.rs:800-838 TL1 payload, hadamard.rs:96-110 vectors, qwen35.rs:241-259).

    python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
import oracle as orc  # noqa: E402


def bf16(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def f32(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def main():
    # 1. TL1 matvec on the reference's 37x384 payload (ops.rs:800-838).
    out_len, in_len = 37, 384
    rb = in_len // 128 * 28
    i = np.arange(out_len * rb, dtype=np.uint64)
    payload = ((i * (0x9B ^ (i >> 7))) & 0xFF).astype(np.uint8)
    g = payload.reshape(-1, 28)
    g[:, 26], g[:, 27] = 0x10, 0x38
    x = (((np.arange(in_len) % 7) - 3.0) * 0.5).astype(np.float32)
    np.savez(HERE / "tl1_matvec_37x384.npz", payload=payload, x=x, out_len=out_len, in_len=in_len,
             y_scalar=orc.matvec_tl1(payload, out_len, in_len, x, simd=0),
             y_sse=orc.matvec_tl1(payload, out_len, in_len, x, simd=1))

    # 2. Ternary GEMM in bitnet.cpp's I2_S / I8_S format: 3 columns of a
    #    40x512 ternary matrix (w_scale 1.5), the int8 rows, the exact sums,
    #    the outputs and this library's tiled repack of the codes.  These
    #    outputs come from the oracle's transcription of the published
    #    bitnet.cpp source, not from bitnet.cpp (its submodule is empty in
    #    the reference): a regression fixture, not a reference vector.
    rng = np.random.default_rng(20261201)
    w = rng.integers(-1, 2, size=(40, 512)).astype(np.int8)
    xa = rng.standard_normal((3, 512)).astype(np.float32)
    xa[1, 7] = 40.0  # an outlier row
    xa[2, :] = xa[2, :] * 1e-6  # a row below the 1e-5 amax floor
    i2s = orc.quantize_i2_s((w * np.float32(1.5)).astype(np.float32))
    xq, s = orc.act_quant_i8(xa)
    acc, y = orc.gemm_i2s(i2s, 40, 512, xq, s)
    np.savez(HERE / "i2s_gemm_40x512x3.npz", i2s=i2s, x=xa, xq=xq, act_scale=s, acc=acc, y=y,
             tiled=orc.i2_tile(orc.i2s_to_canonical(i2s, 40, 512), 40, 512))

    # 3. Hadamard: the reference vectors (hadamard.rs:96-126) and a 2x4096 bf16 case.
    n = 16
    hx = np.array([((k * 11) % 7) - 3.0 for k in range(n)], np.float32)
    hs = np.array([-1.0 if k % 3 == 0 else 1.0 for k in range(n)], np.float32)
    fwd = hx.copy()
    orc.rotate_fwd(fwd, hs, 16)
    ix = np.array([((k * 5) % 9) - 4.0 for k in range(n)], np.float32)
    isg = np.array([-1.0 if k % 4 == 0 else 1.0 for k in range(n)], np.float32)
    inv = ix.copy()
    orc.rotate_inv(inv, isg, 16)
    xb = bf16(rng.standard_normal((2, 4096)).astype(np.float32) * np.where(rng.random((2, 4096)) < 0.01, 50, 1))
    r = f32(xb).copy()
    orc.rotate_rows(r, None, 4096)
    np.savez(HERE / "hadamard.npz", fwd_x=hx, fwd_signs=hs, fwd_y=fwd, inv_x=ix, inv_signs=isg, inv_y=inv,
             rows_x_bf16=xb, rows_y_f32=r, rows_y_bf16=bf16(r))

    # 4. Delta-net: one decode step (B=1, Hk=1, Hv=2) and a 70-token prefill.
    B, Hk, Hv, d = 1, 1, 2, 128
    st = (0.02 * rng.standard_normal((B, Hv, d * d))).astype(np.float32)
    q = bf16(rng.standard_normal((B, Hk, d)).astype(np.float32))
    k = bf16(rng.standard_normal((B, Hk, d)).astype(np.float32))
    v = bf16(rng.standard_normal((B, Hv, d)).astype(np.float32))
    gate = (-np.log1p(np.exp(rng.standard_normal((B, Hv))))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((B, Hv))))).astype(np.float32)
    s_out = st.copy()
    o = orc.gdn_decode(s_out, f32(q), f32(k), f32(v), gate, beta, B, Hk, Hv, d, 3, 1e-6)
    np.savez(HERE / "gdn_decode_b1.npz", state=st, q=q, k=k, v=v, gate=gate, beta=beta, out=o, state_out=s_out)
    T = 70
    st1 = (0.02 * rng.standard_normal((Hv, d * d))).astype(np.float32)
    q = bf16(rng.standard_normal((T, Hk, d)).astype(np.float32))
    k = bf16(rng.standard_normal((T, Hk, d)).astype(np.float32))
    v = bf16(rng.standard_normal((T, Hv, d)).astype(np.float32))
    gate = (-np.log1p(np.exp(rng.standard_normal((T, Hv))))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, Hv))))).astype(np.float32)
    s1 = st1.copy()
    o1 = orc.gdn_prefill_tokens(s1, f32(q), f32(k), f32(v), gate, beta, T, Hk, Hv, d, 3, 1e-6)
    np.savez(HERE / "gdn_prefill_t70.npz", state=st1, q=q, k=k, v=v, gate=gate, beta=beta, out=o1, state_out=s1)


if __name__ == "__main__":
    main()

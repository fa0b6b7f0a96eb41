"""CPU oracle - TEST INFRASTRUCTURE ONLY.

numpy wrappers over ``libouro_oracle.so``, the plain-C restatement of the
reference CPU arithmetic (cluster/src/infer/{dequant,ops,hadamard,qwen35}.rs;
see ouro_oracle.h for the file:line of every function).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the
checker; the product (ouroboros_amd, libouro_hip.so) never does.

Parity status of each function (how it is pinned, tests/test_oracle_*.py):
  f16/bf16 decode, tl1_group, tq1_block ... reference KATs (dequant.rs tests)
  matvec_tl1 / matmul_tl1 .................. reference equivalence tests
                                             (ops.rs:720-750, 800-838)
  rotate_fwd / rotate_inv .................. Sylvester matrix, round trip,
                                             norm, block independence
                                             (hadamard.rs:96-172)
  delta_head_dim ........................... qwen35.rs KATs + float64
                                             brute force
  I2_S pack / I8_S act quant / gemm ........ bitnet.cpp's published rules
                                             (third-party, absent from the
                                             reference checkout): hand KATs of
                                             bytes, ties, the amax floor and
                                             the epilogue; brute force;
                                             invariants
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libouro_oracle.so"

L2NORM_QK, SCALE_Q, KHEAD_DIV = 1, 2, 4
KIND_F32, KIND_F16, KIND_BF16, KIND_TQ1_0, KIND_TL1, KIND_I2_S, KIND_I2 = 0, 1, 30, 34, 143, 36, 0x4932
KIND_Q8_0, KIND_Q3K, KIND_Q4K, KIND_Q5K, KIND_Q6K = 8, 11, 12, 13, 14

_lib: C.CDLL | None = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        h = C.CDLL(str(LIB))
        vp, sz, i32, f32, u32 = C.c_void_p, C.c_size_t, C.c_int, C.c_float, C.c_uint
        sig = {
            "orc_f16_to_f32": (f32, [C.c_uint16]),
            "orc_bf16_to_f32": (f32, [C.c_uint16]),
            "orc_f32_to_bf16_rne": (C.c_uint16, [f32]),
            "orc_tl1_group": (None, [vp, vp]),
            "orc_dequant_tl1_row": (None, [vp, sz, sz, vp]),
            "orc_tq1_block": (None, [vp, vp]),
            "orc_dequant_tq1_row": (None, [vp, sz, sz, vp]),
            "orc_q8_block": (None, [vp, vp]),
            "orc_q4k_block": (None, [vp, vp]),
            "orc_q3k_block": (None, [vp, vp]),
            "orc_q5k_block": (None, [vp, vp]),
            "orc_q6k_block": (None, [vp, vp]),
            "orc_dequant_qblock_row": (i32, [i32, vp, sz, sz, vp]),
            "orc_matvec_qblock": (i32, [vp, i32, sz, sz, vp, vp, i32]),
            "orc_row_bytes": (sz, [i32, sz]),
            "orc_kind_supported": (i32, [u32]),
            "orc_dot": (f32, [vp, vp, sz]),
            "orc_matvec_tl1": (None, [vp, sz, sz, vp, vp, i32, i32]),
            "orc_matmul_tl1": (None, [vp, sz, sz, vp, sz, vp, i32, i32]),
            "orc_matvec_tq1": (None, [vp, sz, sz, vp, vp, i32]),
            "orc_matvec_dense": (None, [vp, i32, sz, sz, vp, vp]),
            "orc_matvec_q": (i32, [vp, i32, sz, sz, vp, vp, i32]),
            "orc_matmul_q": (i32, [vp, i32, sz, sz, vp, sz, vp, i32]),
            "orc_i2_pack": (i32, [vp, sz, sz, vp]),
            "orc_i2_unpack": (None, [vp, sz, sz, vp]),
            "orc_act_quant_i8": (None, [vp, sz, sz, vp, vp]),
            "orc_i2s_bytes": (sz, [sz, sz]),
            "orc_quantize_i2_s": (i32, [vp, sz, sz, vp]),
            "orc_i2s_pack": (i32, [vp, sz, sz, f32, vp]),
            "orc_i2s_code": (i32, [vp, sz, sz, sz]),
            "orc_i2s_scale": (f32, [vp, sz, sz]),
            "orc_quantize_row_i8_s": (None, [vp, sz, vp, vp, vp]),
            "orc_vec_dot_i2_i8_s": (C.c_int32, [vp, sz, sz, vp]),
            "orc_gemm_i2s": (None, [vp, sz, sz, vp, vp, sz, vp, vp, i32]),
            "orc_i2s_to_canonical": (i32, [vp, sz, sz, vp]),
            "orc_i2_tiled_bytes": (sz, [sz, sz]),
            "orc_i2_tile": (sz, [vp, sz, sz, vp]),
            "orc_i2_mfma_bytes": (sz, [sz, sz]),
            "orc_i2_tile_mfma": (sz, [vp, sz, sz, vp]),
            "orc_gemm_i2": (None, [vp, sz, sz, vp, vp, sz, f32, vp, vp, i32]),
            "orc_wht_inplace": (None, [vp, sz]),
            "orc_rotate_fwd": (i32, [vp, vp, sz, sz]),
            "orc_rotate_inv": (i32, [vp, vp, sz, sz]),
            "orc_rotate_rows": (i32, [vp, vp, sz, sz, sz, i32, i32]),
            "orc_delta_head_dim": (None, [vp, sz, vp, vp, vp, f32, f32, vp]),
            "orc_l2_norm": (None, [vp, sz, f32]),
            "orc_softplus": (f32, [f32]),
            "orc_sigmoid": (f32, [f32]),
            "orc_silu": (f32, [f32]),
            "orc_conv_step": (f32, [vp, vp, f32]),
            "orc_gated_norm_rms": (None, [vp, vp, vp, sz, f32, vp]),
            "orc_delta_q_scale": (f32, [sz]),
            "orc_gdn_decode": (None, [vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, u32, f32, i32]),
            "orc_gdn_layer_decode": (None, [vp] * 11 + [sz, sz, sz, sz, u32, f32, i32]),
            "orc_finite_argmax": (sz, [vp, sz]),
            "orc_gdn_prefill_tokens": (None, [vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, u32, f32, i32]),
            "orc_gdn_prefill_varlen": (None, [vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, u32, f32, i32]),
            "orc_mt_threads": (i32, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def f16_to_f32(bits: int) -> float:
    return lib().orc_f16_to_f32(bits)


def bf16_to_f32(bits: int) -> float:
    return lib().orc_bf16_to_f32(bits)


def tl1_group(g28: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g28, dtype=np.uint8)
    out = np.empty(128, np.float32)
    lib().orc_tl1_group(_p(g), _p(out))
    return out


def tq1_block(b54: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b54, dtype=np.uint8)
    out = np.empty(256, np.float32)
    lib().orc_tq1_block(_p(b), _p(out))
    return out


def dequant_tl1_row(payload: np.ndarray, row: int, in_len: int) -> np.ndarray:
    p = np.ascontiguousarray(payload, dtype=np.uint8)
    out = np.empty(in_len, np.float32)
    lib().orc_dequant_tl1_row(_p(p), row, in_len, _p(out))
    return out


def dequant_tq1_row(payload: np.ndarray, row: int, in_len: int) -> np.ndarray:
    p = np.ascontiguousarray(payload, dtype=np.uint8)
    out = np.empty(in_len, np.float32)
    lib().orc_dequant_tq1_row(_p(p), row, in_len // 256 * 54, _p(out))
    return out


# Block bytes / elements of the block-quantised kinds (QuantKind::block_bytes,
# block_elems, dequant.rs:350-372), keyed by ggml dtype id.
QBLOCK = {34: (54, 256), 8: (34, 32), 11: (110, 256), 12: (144, 256), 13: (176, 256), 14: (210, 256)}
_QBLOCK_FN = {8: "orc_q8_block", 11: "orc_q3k_block", 12: "orc_q4k_block", 13: "orc_q5k_block",
              14: "orc_q6k_block", 34: "orc_tq1_block"}


def qblock(kind: int, blk: np.ndarray) -> np.ndarray:
    """Decode one block of a block-quantised kind (q8_block, q4k_block, ...)."""
    bb, be = QBLOCK[kind]
    b = np.ascontiguousarray(blk, dtype=np.uint8)
    assert b.size == bb
    out = np.empty(be, np.float32)
    getattr(lib(), _QBLOCK_FN[kind])(_p(b), _p(out))
    return out


def dequant_qblock(kind: int, payload: np.ndarray) -> np.ndarray:
    """A whole payload of blocks, decoded (dequant_q8_0, dequant_q4_k, ...)."""
    bb, be = QBLOCK[kind]
    p = np.ascontiguousarray(payload, dtype=np.uint8).reshape(-1)
    assert p.size % bb == 0
    nb = p.size // bb
    out = np.empty(nb * be, np.float32)
    if nb:
        lib().orc_dequant_qblock_row(kind, _p(p), 0, p.size, _p(out))
    return out


def row_bytes(kind: int, k: int) -> int:
    return int(lib().orc_row_bytes(kind, k))


def matvec_tl1(payload, out_len, in_len, x, simd=1, nthreads=0) -> np.ndarray:
    p = np.ascontiguousarray(payload, dtype=np.uint8)
    x = _f32(x)
    y = np.empty(out_len, np.float32)
    lib().orc_matvec_tl1(_p(p), out_len, in_len, _p(x), _p(y), simd, nthreads)
    return y


def matmul_tl1(payload, out_len, in_len, x, k, simd=1, nthreads=0) -> np.ndarray:
    p = np.ascontiguousarray(payload, dtype=np.uint8)
    x = _f32(x)
    y = np.empty(k * out_len, np.float32)
    lib().orc_matmul_tl1(_p(p), out_len, in_len, _p(x), k, _p(y), simd, nthreads)
    return y


def matvec_q(payload, kind, out_len, in_len, x, nthreads=0) -> np.ndarray:
    p = np.ascontiguousarray(payload, dtype=np.uint8)
    x = _f32(x)
    y = np.empty(out_len, np.float32)
    if lib().orc_matvec_q(_p(p), kind, out_len, in_len, _p(x), _p(y), nthreads):
        raise ValueError(f"oracle matvec_q: kind {kind} not restated")
    return y


def matmul_q(payload, kind, out_len, in_len, x, k, nthreads=0) -> np.ndarray:
    p = np.ascontiguousarray(payload, dtype=np.uint8)
    x = _f32(x)
    y = np.empty(k * out_len, np.float32)
    if lib().orc_matmul_q(_p(p), kind, out_len, in_len, _p(x), k, _p(y), nthreads):
        raise ValueError(f"oracle matmul_q: kind {kind} not restated")
    return y


def i2_pack(w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.int8)
    out = np.empty((w.shape[0], w.shape[1] // 4), np.uint8)
    if lib().orc_i2_pack(_p(w), w.shape[0], w.shape[1], _p(out)):
        raise ValueError("oracle i2_pack: bad weights or shape")
    return out


def i2_unpack(packed: np.ndarray, out_len: int, in_len: int) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    w = np.empty((out_len, in_len), np.int8)
    lib().orc_i2_unpack(_p(p), out_len, in_len, _p(w))
    return w


def i2_tile(canonical: np.ndarray, out_len: int, in_len: int) -> np.ndarray:
    c = np.ascontiguousarray(canonical, dtype=np.uint8)
    n = int(lib().orc_i2_tiled_bytes(out_len, in_len))
    if n == 0:
        raise ValueError("i2_tile: in_len must be a multiple of 256")
    out = np.empty(n, np.uint8)
    lib().orc_i2_tile(_p(c), out_len, in_len, _p(out))
    return out


def i2_tile_mfma(canonical: np.ndarray, out_len: int, in_len: int) -> np.ndarray:
    c = np.ascontiguousarray(canonical, dtype=np.uint8)
    n = int(lib().orc_i2_mfma_bytes(out_len, in_len))
    if n == 0:
        raise ValueError("i2_tile_mfma: in_len must be a multiple of 256")
    out = np.empty(n, np.uint8)
    lib().orc_i2_tile_mfma(_p(c), out_len, in_len, _p(out))
    return out


def act_quant_i8(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """quantize_row_i8_s per row: (int8 rows, act_scale s = 127 / max(amax, 1e-5))."""
    x = _f32(x)
    if x.ndim == 1:
        x = x[None, :]
    q = np.empty(x.shape, np.int8)
    s = np.empty(x.shape[0], np.float32)
    lib().orc_act_quant_i8(_p(x), x.shape[0], x.shape[1], _p(q), _p(s))
    return q, s


def quantize_row_i8_s(x) -> tuple[np.ndarray, float, int]:
    x = _f32(x).reshape(-1)
    q = np.empty(x.size, np.int8)
    s = np.empty(1, np.float32)
    t = np.empty(1, np.int32)
    lib().orc_quantize_row_i8_s(_p(x), x.size, _p(q), _p(s), _p(t))
    return q, s[0], int(t[0])


def i2s_bytes(nrow: int, n_per_row: int) -> int:
    return int(lib().orc_i2s_bytes(nrow, n_per_row))


def quantize_i2_s(src: np.ndarray) -> np.ndarray:
    """quantize_i2_s of a float [nrow][n_per_row] tensor: n/4 code bytes, the fp32 scale, padding."""
    s = _f32(src)
    out = np.empty(i2s_bytes(*s.shape), np.uint8)
    if lib().orc_quantize_i2_s(_p(s), s.shape[0], s.shape[1], _p(out)):
        raise ValueError("quantize_i2_s: element count not a multiple of 128")
    return out


def i2s_pack(w: np.ndarray, w_scale: float) -> np.ndarray:
    """I2_S bytes of ternary w [out][in] with per-tensor scale w_scale (quantize_i2_s of w * w_scale)."""
    w = np.ascontiguousarray(w, dtype=np.int8)
    out = np.empty(i2s_bytes(*w.shape), np.uint8)
    if lib().orc_i2s_pack(_p(w), w.shape[0], w.shape[1], float(w_scale), _p(out)):
        raise ValueError("i2s_pack: bad weights, scale or shape")
    return out


def i2s_code(i2s, n_per_row: int, r: int, k: int) -> int:
    p = np.ascontiguousarray(i2s, dtype=np.uint8)
    return int(lib().orc_i2s_code(_p(p), n_per_row, r, k))


def i2s_scale(i2s, nrow: int, n_per_row: int) -> float:
    p = np.ascontiguousarray(i2s, dtype=np.uint8)
    return float(lib().orc_i2s_scale(_p(p), nrow, n_per_row))


def i2s_to_canonical(i2s, out_len: int, in_len: int) -> np.ndarray:
    p = np.ascontiguousarray(i2s, dtype=np.uint8)
    out = np.empty((out_len, in_len // 4), np.uint8)
    if lib().orc_i2s_to_canonical(_p(p), out_len, in_len, _p(out)):
        raise ValueError("i2s_to_canonical: bad shape")
    return out


def vec_dot_i2_i8_s(i2s, n_per_row: int, r: int, q) -> int:
    p = np.ascontiguousarray(i2s, dtype=np.uint8)
    q = np.ascontiguousarray(q, dtype=np.int8)
    return int(lib().orc_vec_dot_i2_i8_s(_p(p), n_per_row, r, _p(q)))


def gemm_i2s(i2s, out_len, in_len, xq, act_scale, nthreads=0):
    """bitnet.cpp's I2_S mul_mat: returns (acc = sum w*q, y) in column-major [ncols][out_len]."""
    p = np.ascontiguousarray(i2s, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.int8).reshape(-1, in_len)
    s = _f32(act_scale).reshape(-1)
    nc = xq.shape[0]
    acc = np.empty(nc * out_len, np.int32)
    y = np.empty(nc * out_len, np.float32)
    lib().orc_gemm_i2s(_p(p), out_len, in_len, _p(xq), _p(s), nc, _p(acc), _p(y), nthreads)
    return acc, y


def gemm_i2(packed, out_len, in_len, xq, act_scale, w_scale, nthreads=0):
    """Canonical codes with bitnet.cpp's epilogue: (acc, y = (acc / s) * w_scale)."""
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.int8).reshape(-1, in_len)
    ds = _f32(act_scale).reshape(-1)
    nc = xq.shape[0]
    acc = np.empty(nc * out_len, np.int32)
    y = np.empty(nc * out_len, np.float32)
    lib().orc_gemm_i2(_p(p), out_len, in_len, _p(xq), _p(ds), nc, float(w_scale), _p(acc), _p(y),
                      nthreads)
    return acc, y


def wht_inplace(x: np.ndarray) -> None:
    assert x.dtype == np.float32 and x.flags.c_contiguous
    lib().orc_wht_inplace(_p(x), x.size)


def rotate_fwd(x: np.ndarray, signs, block: int) -> None:
    assert x.dtype == np.float32 and x.flags.c_contiguous
    s = _f32(signs)
    if lib().orc_rotate_fwd(_p(x), _p(s), x.size, block):
        raise ValueError("rotate_fwd: check_args failed")


def rotate_inv(x: np.ndarray, signs, block: int) -> None:
    assert x.dtype == np.float32 and x.flags.c_contiguous
    s = _f32(signs)
    if lib().orc_rotate_inv(_p(x), _p(s), x.size, block):
        raise ValueError("rotate_inv: check_args failed")


def rotate_rows(x: np.ndarray, signs, block: int, inverse=False, nthreads=0) -> None:
    assert x.dtype == np.float32 and x.flags.c_contiguous and x.ndim == 2
    s = _f32(signs) if signs is not None else np.ones(x.shape[1], np.float32)
    if lib().orc_rotate_rows(_p(x), _p(s), x.shape[0], x.shape[1], block, int(inverse), nthreads):
        raise ValueError("rotate_rows: check_args failed")


def delta_head_dim(state: np.ndarray, sdim: int, q, k, v, gate: float, beta: float,
                   out: np.ndarray) -> None:
    assert state.dtype == np.float32 and state.flags.c_contiguous
    q, k, v = _f32(q), _f32(k), _f32(v)
    assert out.dtype == np.float32 and out.flags.c_contiguous
    lib().orc_delta_head_dim(_p(state), sdim, _p(q), _p(k), _p(v), gate, beta, _p(out))


def l2_norm(v: np.ndarray, eps: float) -> None:
    assert v.dtype == np.float32 and v.flags.c_contiguous
    lib().orc_l2_norm(_p(v), v.size, eps)


def softplus(x: float) -> float:
    return lib().orc_softplus(x)


def sigmoid(x: float) -> float:
    return lib().orc_sigmoid(x)


def silu(x: float) -> float:
    return lib().orc_silu(x)


def conv_step(ring: np.ndarray, w, x: float) -> float:
    assert ring.dtype == np.float32 and ring.size == 3
    w = _f32(w)
    return lib().orc_conv_step(_p(ring), _p(w), x)


def gated_norm_rms(x, w, gate, eps) -> np.ndarray:
    x, w, gate = _f32(x), _f32(w), _f32(gate)
    y = np.empty_like(x)
    lib().orc_gated_norm_rms(_p(x), _p(w), _p(gate), x.size, eps, _p(y))
    return y


def delta_q_scale(d: int = 128) -> float:
    return lib().orc_delta_q_scale(d)


def gdn_decode(state, q, k, v, gate, beta, B, Hk, Hv, d, flags, eps, nthreads=0) -> np.ndarray:
    assert state.dtype == np.float32 and state.flags.c_contiguous
    q, k, v, gate, beta = _f32(q), _f32(k), _f32(v), _f32(gate), _f32(beta)
    out = np.empty((B, Hv, d), np.float32)
    lib().orc_gdn_decode(_p(state), _p(q), _p(k), _p(v), _p(gate), _p(beta), _p(out), B, Hk, Hv, d,
                         flags, eps, nthreads)
    return out


def gdn_prefill_tokens(state, q, k, v, gate, beta, T, Hk, Hv, d, flags, eps, nthreads=0):
    assert state.dtype == np.float32 and state.flags.c_contiguous
    q, k, v, gate, beta = _f32(q), _f32(k), _f32(v), _f32(gate), _f32(beta)
    out = np.empty((T, Hv, d), np.float32)
    lib().orc_gdn_prefill_tokens(_p(state), _p(q), _p(k), _p(v), _p(gate), _p(beta), _p(out), T, Hk,
                                 Hv, d, flags, eps, nthreads)
    return out


def gdn_prefill_varlen(state, q, k, v, gate, beta, cu_seqlens, Hk, Hv, d, flags, eps, nthreads=0):
    """Token-loop prefill of N packed sequences (state [N][Hv][d*d], updated in place)."""
    assert state.dtype == np.float32 and state.flags.c_contiguous
    q, k, v, gate, beta = _f32(q), _f32(k), _f32(v), _f32(gate), _f32(beta)
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    T, N = int(cu[-1]), len(cu) - 1
    out = np.empty((T, Hv, d), np.float32)
    lib().orc_gdn_prefill_varlen(_p(state), _p(q), _p(k), _p(v), _p(gate), _p(beta), _p(out), _p(cu), N, Hk,
                                 Hv, d, flags, eps, nthreads)
    return out


GDN_V_GROUPED = 8


def gdn_layer_decode(qkv, z, beta_raw, alpha_raw, dt_bias, a_log, conv_w, norm_w, conv, state, B, Hk, Hv, d,
                     flags, eps, nthreads=0) -> np.ndarray:
    """run_delta's layer block (qwen35.rs:1066-1140); conv and state are updated in place."""
    for a in (conv, state):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    args = [_f32(x) for x in (qkv, z, beta_raw, alpha_raw, dt_bias, a_log, conv_w, norm_w)]
    out = np.empty((B, Hv * d), np.float32)
    lib().orc_gdn_layer_decode(*(_p(x) for x in args), _p(conv), _p(state), _p(out), B, Hk, Hv, d, flags, eps,
                               nthreads)
    return out


def finite_argmax(l) -> int:
    """infer/mod.rs:70-83."""
    a = _f32(l)
    return int(lib().orc_finite_argmax(_p(a), a.size))


def mt_threads() -> int:
    return int(lib().orc_mt_threads())


def nproc() -> int:
    return os.cpu_count() or 1

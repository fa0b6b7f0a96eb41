#!/usr/bin/env python3
"""Benchmark of the quantized-inference hot path on one MI355X.

Headline (`value`): ternary GEMV GB/s on the 6912x2560 I2 layer (2-bit
weights, int8 per-token-absmax activations, fp32 output).  One step is one
grouped launch over 256 distinct weight matrices (1.14 GB, 4.5x the 256 MB
last-level cache, so every byte comes from HBM), inputs resident in HBM.
The same launch over 64 matrices (285 MB, about the cache's size) is
reported beside it.  Also measured, reported under
"secondary": gated delta-net decode (B=32, Hk=16, Hv=32, d=128, fp32 state,
8 rotating state sets = 512 MiB) in tokens/s, the 512x4096 bf16
Walsh-Hadamard rotation in GB/s, the chunked prefill of 4 x 4096 tokens in
tokens/s and TFLOP/s, the ternary GEMM at 4..2048 columns, the TL1 lm_head
GEMV, the hybrid stack (24 layers, 64 ragged prompts of 16..2048 tokens then
128 greedy decode steps) in tokens/s with its decode step against the HBM
roofline, and a 512 MiB device copy as the bandwidth reference.

Every kernel time comes from HIP events recorded on the stream the kernels
run on: the null stream, where back-to-back launches carry no extra gap.
The CPU baseline is the oracle (a C restatement of the reference's
threaded CPU kernels) on a bounded sample, rank 0 only.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
METRIC = "ternary GEMV GB/s (% HBM peak); gated delta-net decode tokens/sec, 1 GPU"

# Algorithmic bytes per unit (weights + int8 x + x scale + w scale + fp32 y).
GEMV_OUT, GEMV_IN, GEMV_MATS, GEMV_MATS_SMALL = 6912, 2560, 256, 64
GEMV_BYTES = GEMV_OUT * GEMV_IN // 4 + GEMV_IN + 4 + 4 + GEMV_OUT * 4  # 4,453,896
# GDN decode step: state read+write, q,k bf16, v bf16, gate+beta f32, out f32.
GDN_B, GDN_HK, GDN_HV, GDN_D, GDN_SETS = 32, 16, 32, 128, 8
GDN_BYTES = (2 * GDN_B * GDN_HV * GDN_D * GDN_D * 4 + 2 * GDN_B * GDN_HK * GDN_D * 2
             + GDN_B * GDN_HV * GDN_D * 2 + 2 * GDN_B * GDN_HV * 4 + GDN_B * GDN_HV * GDN_D * 4)
# FWHT 512 x 4096 bf16 in and out.
FW_ROWS, FW_N, FW_BUFS = 512, 4096, 32
FW_BYTES = 2 * FW_ROWS * FW_N * 2
# fused int8 epilogue: bf16 in, int8 rows and one fp32 scale per row out
FW_Q_BYTES = FW_ROWS * FW_N * 2 + FW_ROWS * FW_N + FW_ROWS * 4
# Chunked prefill: 4 sequences x 4096 tokens, chunk 64, same heads.
PF_SEQ, PF_LEN, PF_C = 4, 4096, 64
PF_T = PF_SEQ * PF_LEN
# Each contraction counted once per (chunk, v-head): K K^T, Q K^T (64x64x128),
# K S0, Q S0 (64x128x128), T R, Pt U (64x64x128), K^T U (128x64x128).
PF_FLOP_CHUNK_HEAD = 2 * (64 * 64 * 128 * 4 + 64 * 128 * 128 * 2 + 128 * 64 * 128)
PF_FLOPS = PF_FLOP_CHUNK_HEAD * (PF_LEN // PF_C) * PF_SEQ * GDN_HV
# q,k,v bf16 in, gate+beta f32 in, out f32, state in+out.
PF_BYTES = (2 * PF_T * GDN_HK * GDN_D * 2 + PF_T * GDN_HV * GDN_D * 2 + 2 * PF_T * GDN_HV * 4
            + PF_T * GDN_HV * GDN_D * 4 + 2 * PF_SEQ * GDN_HV * GDN_D * GDN_D * 4)
MFMA_BF16_PEAK_TFLOPS = 2500.0
# Ternary x int8 GEMM (K-column matmul) on the 6912x2560 layer.
GM_OUT, GM_IN, GM_COLS_MAIN = 6912, 2560, 2048
GM_COLS = (4, 8, 16, 64, 512, GM_COLS_MAIN)
INT8_MFMA_PEAK_TOPS = 5000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


BOX_CPU_SHARE = 16  # host threads one GPU's job may keep busy on the GPU hosts


def available_parallelism() -> tuple[int, dict]:
    """Rust's std::thread::available_parallelism, the reference's default
    thread count (mt_threads, ops.rs:62-73): the CPUs this process may run on
    (its affinity mask), bounded by a cgroup v2 CPU quota when one is set."""
    info = {"nproc": os.cpu_count() or 1}
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    info["affinity_cpus"] = n
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            q = max(1, -(-int(quota) // int(period)))
            info["cgroup_quota_cpus"] = q
            n = min(n, q)
    except (OSError, ValueError):
        pass
    return n, info


def cpu_threads() -> tuple[int, dict]:
    """OURO_N_THREADS, else available_parallelism (ops.rs:62-73), at most the
    GPU host's per-job CPU share (recorded when it applies)."""
    n, info = available_parallelism()
    env = os.environ.get("OURO_N_THREADS")
    if env and env.isdigit() and int(env) > 0:
        info["source"] = "OURO_N_THREADS"
        return int(env), info
    info["source"] = "available_parallelism"
    if n > BOX_CPU_SHARE:
        info["capped_from"] = n
        info["cap_reason"] = f"{BOX_CPU_SHARE} threads: the CPU share of one GPU's job on the GPU host"
        n = BOX_CPU_SHARE
    return n, info


def cpu_median(fn, warmup: int = 3, min_runs: int = 10, budget_s: float = 4.0, max_runs: int = 200):
    """Median wall time of fn() over >= min_runs runs after `warmup` untimed ones
    (more runs while the budget lasts); returns (seconds, runs)."""
    for _ in range(warmup):
        fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t_start < budget_s and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def time_events(stream, fn, steps: int, warmup: int, min_warm_s: float = 0.15) -> float:
    """Average ms per call of fn() on `stream`, HIP events around `steps` calls.

    Untimed warm-up: `warmup` calls, then more until `min_warm_s` of wall time
    has passed, so the GPU clocks have ramped before the timed region."""
    from ouroboros_amd._lib import call
    from ouroboros_amd.device import Event, synchronize

    t0 = time.perf_counter()
    i = 0
    while i < warmup or time.perf_counter() - t0 < min_warm_s:
        fn(i)
        i += 1
        if i % 16 == 0:
            synchronize(stream)
    synchronize(stream)
    call("ouro_device_synchronize")
    e0, e1 = Event(), Event()
    e0.record(stream)
    for i in range(steps):
        fn(warmup + i)
    e1.record(stream)
    call("ouro_device_synchronize")
    return e0.elapsed_ms(e1) / steps


def bench_gemv(stream, steps, warmup, orc):
    from ouroboros_amd import ops, quant
    from ouroboros_amd._lib import call
    from ouroboros_amd.device import DeviceBuffer

    rng = np.random.default_rng(1234)
    tb = ops.i2_tiled_bytes(GEMV_OUT, GEMV_IN)
    stride = (tb + 4 + 255) // 256 * 256
    w_all = DeviceBuffer((GEMV_MATS * stride,), np.uint8)
    n_distinct = 4  # distinct contents, copied to GEMV_MATS distinct addresses
    tensors, scales = [], []
    for m in range(n_distinct):
        # trits i.i.d. with p = 1/3 each, w_scale ~ U(0.5, 2), as bitnet.cpp I2_S tensors
        w = rng.integers(-1, 2, size=(GEMV_OUT, GEMV_IN)).astype(np.int8)
        scales.append(np.float32(rng.uniform(0.5, 2.0)))
        tensors.append(quant.i2s_pack(w, scales[-1]))
    # repacked on the device to the tiled layout, as a resident upload does
    payloads = [ops.i2s_payload(t, GEMV_OUT, GEMV_IN) for t in tensors]
    for m in range(GEMV_MATS):
        call("ouro_memcpy_dtod", w_all.ptr + m * stride, payloads[m % n_distinct].ptr, tb + 4, None)
    x = rng.standard_normal((GEMV_MATS, GEMV_IN)).astype(np.float32)
    xd = DeviceBuffer.from_host(x)
    xq = DeviceBuffer((GEMV_MATS, GEMV_IN), np.int8)
    ds = DeviceBuffer((GEMV_MATS,), np.float32)
    ops.act_quant_i8(xd, GEMV_MATS, GEMV_IN, xq, ds, stream)
    wsc = DeviceBuffer.from_host(np.array([scales[m % n_distinct] for m in range(GEMV_MATS)], np.float32))
    y = DeviceBuffer((GEMV_MATS, GEMV_OUT), np.float32)
    call("ouro_device_synchronize")

    def grouped(_i, count=GEMV_MATS):
        call("ouro_gemv_i2_grouped", w_all.ptr, stride, wsc.ptr, xq.ptr, GEMV_IN, ds.ptr, y.ptr,
             GEMV_OUT, GEMV_OUT, GEMV_IN, count, stream)

    ms_small = time_events(stream, lambda i: grouped(i, GEMV_MATS_SMALL), steps, warmup)
    ms = time_events(stream, grouped, steps, warmup)

    # parity spot check of the timed output (not timed): matrix 0 and 5
    got = y.download()
    if orc is not None:
        xq_h, ds_h = xq.download(), ds.download()
        for m in (0, 5):
            _, want = orc.gemm_i2s(tensors[m % n_distinct], GEMV_OUT, GEMV_IN, xq_h[m:m + 1], ds_h[m:m + 1])
            if not np.array_equal(got[m].view(np.uint32), want.view(np.uint32)):
                raise SystemExit(f"GEMV parity failure on matrix {m}")

    # single-matrix launches back to back (each a different matrix)
    def single(i):
        m = i % GEMV_MATS
        call("ouro_gemm_i2", w_all.ptr + m * stride, GEMV_OUT, GEMV_IN, wsc.ptr + 4 * m,
             xq.ptr + m * GEMV_IN, ds.ptr + 4 * m, 1, y.ptr + 4 * m * GEMV_OUT, None, stream)

    ms_single = time_events(stream, single, 4 * GEMV_MATS, GEMV_MATS)
    return ms, ms_single, ms_small


def bench_gdn(stream, steps, warmup):
    from ouroboros_amd import quant, qwen35
    from ouroboros_amd._lib import GDN_L2NORM_QK, GDN_SCALE_Q, call
    from ouroboros_amd.device import DeviceBuffer

    rng = np.random.default_rng(99)
    B, Hk, Hv, d = GDN_B, GDN_HK, GDN_HV, GDN_D
    per = B * Hv * d * d
    states = DeviceBuffer((GDN_SETS, per), np.float32)
    init = (0.02 * rng.standard_normal(per)).astype(np.float32)
    for s in range(GDN_SETS):
        call("ouro_memcpy_htod", states.ptr + 4 * s * per, init.ctypes.data, 4 * per)
    q = DeviceBuffer.from_host(quant.f32_to_bf16_bits(rng.standard_normal((B, Hk, d)).astype(np.float32)))
    k = DeviceBuffer.from_host(quant.f32_to_bf16_bits(rng.standard_normal((B, Hk, d)).astype(np.float32)))
    v = DeviceBuffer.from_host(quant.f32_to_bf16_bits(rng.standard_normal((B, Hv, d)).astype(np.float32)))
    beta = DeviceBuffer.from_host((1 / (1 + np.exp(-rng.standard_normal((B, Hv))))).astype(np.float32))
    gate = DeviceBuffer.from_host((-np.log1p(np.exp(rng.standard_normal((B, Hv))))).astype(np.float32))
    out = DeviceBuffer((B, Hv, d), np.float32)
    fl = GDN_L2NORM_QK | GDN_SCALE_Q

    def step(i):
        s = i % GDN_SETS
        call("ouro_gdn_decode", states.ptr + 4 * s * per, q.ptr, k.ptr, 1, v.ptr, 1, gate.ptr, beta.ptr,
             out.ptr, B, Hk, Hv, d, fl, 1e-6, stream)

    return time_events(stream, step, max(steps, 2 * GDN_SETS), warmup)


LY_CH = 2 * GDN_HK * GDN_D + GDN_HV * GDN_D
# state R+W, conv ring R+W (3 f32 per channel), qkv in, z in, gates in, out; conv and norm weights
LY_BYTES = (2 * GDN_B * GDN_HV * GDN_D * GDN_D * 4 + 2 * GDN_B * LY_CH * 12 + GDN_B * LY_CH * 4
            + 2 * GDN_B * GDN_HV * GDN_D * 4 + 2 * GDN_B * GDN_HV * 4 + LY_CH * 16 + GDN_D * 4 + 2 * GDN_HV * 4)


def bench_layer(stream, steps, warmup):
    """The whole delta-net layer block of a decode step (gates, conv + SiLU,
    recurrence, gated RMS norm) at the decode shape, 8 rotating state sets."""
    from ouroboros_amd import qwen35
    from ouroboros_amd._lib import GDN_V_GROUPED, call
    from ouroboros_amd.device import DeviceBuffer

    rng = np.random.default_rng(17)
    B, Hk, Hv, d = GDN_B, GDN_HK, GDN_HV, GDN_D
    per = B * Hv * d * d
    states = DeviceBuffer((GDN_SETS, per), np.float32)
    init = (0.02 * rng.standard_normal(per)).astype(np.float32)
    for s in range(GDN_SETS):
        call("ouro_memcpy_htod", states.ptr + 4 * s * per, init.ctypes.data, 4 * per)
    f = lambda *sh: DeviceBuffer.from_host(rng.standard_normal(sh).astype(np.float32))  # noqa: E731
    qkv, z, br, ar, dt, nw, conv = f(B, LY_CH), f(B, Hv * d), f(B, Hv), f(B, Hv), f(Hv), f(d), f(B, LY_CH, 3)
    al = DeviceBuffer.from_host((-np.exp(rng.standard_normal(Hv))).astype(np.float32))
    cw = DeviceBuffer.from_host((0.5 * rng.standard_normal((LY_CH, 4))).astype(np.float32))
    out = DeviceBuffer((B, Hv * d), np.float32)
    ws = DeviceBuffer((qwen35.layer_workspace_bytes(B, Hk, Hv, d),), np.uint8)

    def step(i):
        s = i % GDN_SETS
        call("ouro_gdn_layer_decode", qkv.ptr, z.ptr, br.ptr, ar.ptr, dt.ptr, al.ptr, cw.ptr, nw.ptr, conv.ptr,
             states.ptr + 4 * s * per, out.ptr, B, Hk, Hv, d, GDN_V_GROUPED, 1e-6, ws.ptr, stream)

    return time_events(stream, step, max(steps, 2 * GDN_SETS), warmup)


TL1_OUT, TL1_IN = 248320, 5120
TL1_ROW = TL1_IN // 128 * 28
TL1_BYTES = TL1_OUT * TL1_ROW + TL1_IN * 4 + TL1_OUT * 4


def tl1_lmhead_payload():
    """The reference's own lm_head probe input (ops.rs:694-717): bytes
    (i ^ (i >> 13)) * 0x9E, fp16 scale 1.0 in every 28-byte group, x[i] = ((i % 13) - 6) / 10."""
    i = np.arange(TL1_OUT * TL1_ROW, dtype=np.uint32)
    payload = ((i ^ (i >> 13)) * 0x9E).astype(np.uint8)
    g = payload.reshape(-1, 28)
    g[:, 26], g[:, 27] = 0x00, 0x3C
    x = (((np.arange(TL1_IN) % 13) - 6.0) * 0.1).astype(np.float32)
    return payload, x


def bench_tl1(stream, steps, warmup):
    """TL1 (PTQ1_0) matvec at the reference's lm_head probe shape 248320x5120:
    a resident weight handle (repacked on upload for the table-lookup GEMV),
    the same with the fused finite_argmax (greedy sample), the raw-payload
    ouro_matvec_q path, and ouro_matvec_q on a raw TQ1_0 payload of the same
    shape."""
    import ctypes as C

    from ouroboros_amd._lib import KIND_TL1, KIND_TQ1_0, call
    from ouroboros_amd.device import DeviceBuffer

    payload, x = tl1_lmhead_payload()
    h = C.c_void_p()
    call("ouro_weight_upload", KIND_TL1, payload.ctypes.data, payload.nbytes, TL1_OUT, TL1_IN, 1.0, 1, C.byref(h))
    xd = DeviceBuffer.from_host(x)
    y = DeviceBuffer((TL1_OUT,), np.float32)
    idx = DeviceBuffer((1,), np.int32)
    n = max(3, steps // 5)
    ms = time_events(stream, lambda _i: call("ouro_weight_matvec", h.value, xd.ptr, y.ptr, stream), n, 2)
    ms_am = time_events(stream, lambda _i: call("ouro_weight_matvec_argmax", h.value, xd.ptr, None, idx.ptr, stream),
                        n, 2)
    call("ouro_weight_free", h.value)
    w = DeviceBuffer.from_host(payload)
    ms_raw = time_events(stream, lambda _i: call("ouro_matvec_q", w.ptr, KIND_TL1, TL1_OUT, TL1_IN, xd.ptr, y.ptr,
                                                 stream), n, 2)
    del w
    # the same shape as a raw TQ1_0 payload (random bytes, d = 1.0)
    rng = np.random.default_rng(17)
    tq = rng.integers(0, 256, TL1_OUT * (TL1_IN // 256) * 54, dtype=np.uint8)
    g = tq.reshape(-1, 54)
    g[:, 52], g[:, 53] = 0x00, 0x3C
    wq = DeviceBuffer.from_host(tq)
    ms_tq1 = time_events(stream, lambda _i: call("ouro_matvec_q", wq.ptr, KIND_TQ1_0, TL1_OUT, TL1_IN, xd.ptr, y.ptr,
                                                 stream), n, 2)
    del wq
    # K columns from one pass over a resident weight (matmul_tl1, ops.rs:156-286): K = 1 is the lookup
    # matvec, K >= 2 the int8 MFMA pass; the lm_head probe payload and a random 6912x2560 layer
    rng = np.random.default_rng(19)
    small = rng.integers(0, 256, GEMV_OUT * (GEMV_IN // 128) * 28, dtype=np.uint8)
    gs = small.reshape(-1, 28)
    gs[:, 26], gs[:, 27] = 0x00, 0x2C  # d = 1/16
    kcols = []
    for name, pl, out_len, in_len in (("248320x5120 (lm_head probe)", payload, TL1_OUT, TL1_IN),
                                      ("6912x2560", small, GEMV_OUT, GEMV_IN)):
        hk = C.c_void_p()
        call("ouro_weight_upload", KIND_TL1, pl.ctypes.data, pl.nbytes, out_len, in_len, 1.0, 8, C.byref(hk))
        xk = DeviceBuffer.from_host(rng.standard_normal(8 * in_len).astype(np.float32))
        yk = DeviceBuffer((8 * out_len,), np.float32)
        nk = max(3, steps // 5) if out_len == TL1_OUT else steps
        for k in (1, 4, 8):
            t = time_events(stream, lambda _i: call("ouro_weight_matmul", hk.value, xk.ptr, k, yk.ptr, stream), nk, 2)
            kcols.append({"shape": name, "k": k, "us_per_call": round(t * 1e3, 2),
                          "weight_stream_GBs": round(out_len * (in_len // 128) * 28 / (t * 1e-3) / 1e9, 1)})
        call("ouro_weight_free", hk.value)
    # a resident TQ1_0 handle of the lm_head shape (random bytes, d = 1): K = 1 the lookup matvec, K >= 2
    # the same int8 MFMA pass on its trits
    hk = C.c_void_p()
    call("ouro_weight_upload", KIND_TQ1_0, tq.ctypes.data, tq.nbytes, TL1_OUT, TL1_IN, 1.0, 8, C.byref(hk))
    xk = DeviceBuffer.from_host(rng.standard_normal(8 * TL1_IN).astype(np.float32))
    yk = DeviceBuffer((8 * TL1_OUT,), np.float32)
    for k in (1, 4, 8):
        t = time_events(stream, lambda _i: call("ouro_weight_matmul", hk.value, xk.ptr, k, yk.ptr, stream),
                        max(3, steps // 5), 2)
        kcols.append({"shape": "248320x5120 TQ1_0 handle", "k": k, "us_per_call": round(t * 1e3, 2),
                      "weight_stream_GBs": round(tq.nbytes / (t * 1e-3) / 1e9, 1)})
    call("ouro_weight_free", hk.value)
    # the same on the raw payload through ouro_matmul_q (K = 1: the raw lookup matvec)
    w = DeviceBuffer.from_host(payload)
    xk = DeviceBuffer.from_host(rng.standard_normal(8 * TL1_IN).astype(np.float32))
    yk = DeviceBuffer((8 * TL1_OUT,), np.float32)
    for k in (1, 4, 8):
        t = time_events(stream, lambda _i: call("ouro_matmul_q", w.ptr, KIND_TL1, TL1_OUT, TL1_IN, xk.ptr, k, yk.ptr,
                                                stream), max(3, steps // 5), 2)
        kcols.append({"shape": "248320x5120 raw payload (ouro_matmul_q)", "k": k, "us_per_call": round(t * 1e3, 2),
                      "weight_stream_GBs": round(payload.nbytes / (t * 1e-3) / 1e9, 1)})
    return ms, ms_am, ms_raw, ms_tq1, tq.nbytes, kcols


# The block-quantised kinds of matvec_q (Q8_0, Q3_K..Q6_K) on the lm_head
# probe shape and on the 6912x2560 layer (64 rotating copies, ~0.7-1.2 GB).
KQ_KINDS = (("Q8_0", 8, 34, 32), ("Q3_K", 11, 110, 256), ("Q4_K", 12, 144, 256), ("Q5_K", 13, 176, 256),
            ("Q6_K", 14, 210, 256))


def bench_kquant(stream, steps, warmup):
    """ouro_matvec_q on raw ggml blocks (matvec_qblock, ops.rs:101-128):
    random code bytes with f16 scales in a model's range, fp32 x and y."""
    from ouroboros_amd._lib import call
    from ouroboros_amd.device import DeviceBuffer

    rng = np.random.default_rng(23)
    rows = []
    for name, kind, bb, be in KQ_KINDS:
        for out_len, in_len, copies in ((TL1_OUT, TL1_IN, 1), (GEMV_OUT, GEMV_IN, 64)):
            wb = out_len * (in_len // be) * bb
            p = rng.integers(0, 256, wb, dtype=np.uint8)
            blk = p.reshape(-1, bb)
            for o in ({8: [0], 11: [108], 12: [0, 2], 13: [0, 2], 14: [208]}[kind]):
                d = rng.uniform(0.002, 0.02, blk.shape[0]).astype(np.float16).view(np.uint16)
                blk[:, o], blk[:, o + 1] = d & 0xFF, d >> 8
            w = DeviceBuffer((wb * copies,), np.uint8)
            for c in range(copies):  # the same bytes in each copy; each launch reads a different one
                call("ouro_memcpy_htod", w.ptr + c * wb, p.ctypes.data, wb)
            del p, blk
            xd = DeviceBuffer.from_host(rng.standard_normal(in_len).astype(np.float32))
            y = DeviceBuffer((out_len,), np.float32)
            n = max(3, steps // 5) if copies == 1 else steps
            ms = time_events(stream, lambda i: call("ouro_matvec_q", w.ptr + (i % copies) * wb, kind, out_len,
                                                    in_len, xd.ptr, y.ptr, stream), n, 2)
            alg = wb + 4 * (in_len + out_len)
            gbs = alg / (ms * 1e-3) / 1e9
            rows.append({"kind": name, "out_len": out_len, "in_len": in_len, "us_per_call": round(ms * 1e3, 2),
                         "bytes_per_call": alg, "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)})
            del w
    return rows


def bench_gemm(stream, steps, warmup, orc):
    """Ternary x int8 GEMM (the K-column matmul_q, ops.rs:156-230) on the
    6912x2560 layer: the int8 MFMA GEMM (ouro_gemm_i2_mfma) for 4 .. 2048
    columns, and the multi-column GEMV (ouro_gemm_i2) for few columns."""
    from ouroboros_amd import ops, quant
    from ouroboros_amd._lib import call
    from ouroboros_amd.device import DeviceBuffer

    rng = np.random.default_rng(21)
    i2s = quant.i2s_pack(rng.integers(-1, 2, size=(GM_OUT, GM_IN)).astype(np.int8), 1.5)
    p_gemv = ops.i2s_payload(i2s, GM_OUT, GM_IN)
    p_mfma = ops.i2s_mfma_payload(i2s, GM_OUT, GM_IN)
    tb_g, tb_m = ops.i2_tiled_bytes(GM_OUT, GM_IN), ops.i2_mfma_bytes(GM_OUT, GM_IN)
    nmax = max(GM_COLS)
    x = DeviceBuffer.from_host(rng.standard_normal((nmax, GM_IN)).astype(np.float32))
    xq = DeviceBuffer((nmax, GM_IN), np.int8)
    ds = DeviceBuffer((nmax,), np.float32)
    ops.act_quant_i8(x, nmax, GM_IN, xq, ds, stream)
    y = DeviceBuffer((nmax * GM_OUT,), np.float32)
    call("ouro_device_synchronize")
    rows = []
    for n in GM_COLS:
        reps = max(5, min(steps, int(2e5 / (GM_OUT * n / 1e3 + 50))))
        ms_m = time_events(stream, lambda _i: call("ouro_gemm_i2_mfma", p_mfma.ptr, GM_OUT, GM_IN, p_mfma.ptr + tb_m,
                                                   xq.ptr, ds.ptr, n, y.ptr, None, stream), reps, 2)
        row = {"cols": n, "mfma_us": round(ms_m * 1e3, 2),
               "mfma_tops": round(2.0 * GM_OUT * GM_IN * n / (ms_m * 1e-3) / 1e12, 1)}
        if n <= 16:
            ms_v = time_events(stream, lambda _i: call("ouro_gemm_i2", p_gemv.ptr, GM_OUT, GM_IN, p_gemv.ptr + tb_g,
                                                       xq.ptr, ds.ptr, n, y.ptr, None, stream), reps, 2)
            row["gemv_us"] = round(ms_v * 1e3, 2)
        rows.append(row)
    # The vendor's dense int8 GEMM (hipBLASLt through torch._int_mm, 8-bit
    # weights) on the same product, as a reference point for the MFMA rate.
    vendor = None
    try:
        import torch
        if torch.cuda.is_available():
            a8 = torch.randint(-127, 128, (GM_COLS_MAIN, GM_IN), dtype=torch.int8, device="cuda")
            b8 = torch.randint(-127, 128, (GM_IN, GM_OUT), dtype=torch.int8, device="cuda")
            for _ in range(5):
                torch._int_mm(a8, b8)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(20):
                torch._int_mm(a8, b8)
            e1.record()
            torch.cuda.synchronize()
            vendor = e0.elapsed_time(e1) / 20
    except Exception as exc:  # the reference point is optional
        log(f"vendor int8 GEMM reference skipped: {exc}")
    # parity spot check of the MFMA path (not timed): 64 columns against the oracle
    if orc is not None:
        call("ouro_gemm_i2_mfma", p_mfma.ptr, GM_OUT, GM_IN, p_mfma.ptr + tb_m, xq.ptr, ds.ptr, 64, y.ptr, None, stream)
        got = y.download()[:64 * GM_OUT]
        _, want = orc.gemm_i2s(i2s, GM_OUT, GM_IN, xq.download()[:64], ds.download()[:64])
        if not np.array_equal(got.view(np.uint32), want.reshape(-1).view(np.uint32)):
            raise SystemExit("ternary GEMM parity failure")
    return rows, vendor


def bench_fwht(stream, steps, warmup):
    from ouroboros_amd import quant
    from ouroboros_amd._lib import DT_BF16, call
    from ouroboros_amd.device import DeviceBuffer

    rng = np.random.default_rng(7)
    per = FW_ROWS * FW_N
    x = rng.standard_normal(per).astype(np.float32)
    x[rng.random(per) < 0.01] *= 50.0
    xb = quant.f32_to_bf16_bits(x)
    src = DeviceBuffer((FW_BUFS, per), np.uint16)
    dst = DeviceBuffer((FW_BUFS, per), np.uint16)
    for b in range(FW_BUFS):
        call("ouro_memcpy_htod", src.ptr + 2 * b * per, xb.ctypes.data, 2 * per)

    def step(i):
        b = i % FW_BUFS
        call("ouro_fwht_rows", src.ptr + 2 * b * per, DT_BF16, dst.ptr + 2 * b * per, DT_BF16, FW_ROWS,
             FW_N, FW_N, None, 0, None, None, stream)

    ms = time_events(stream, step, max(steps, 2 * FW_BUFS), warmup)

    def whole(_i):  # all 32 buffers as one launch of 16384 rows
        call("ouro_fwht_rows", src.ptr, DT_BF16, dst.ptr, DT_BF16, FW_ROWS * FW_BUFS, FW_N, FW_N, None, 0,
             None, None, stream)

    ms_all = time_events(stream, whole, max(2, steps // 4), 2)

    # the fused epilogue: each rotated row (as bf16) quantised to int8 for the
    # ternary product that follows (quantize_row_i8_s), with and without
    # storing the bf16 rows
    xq = DeviceBuffer((FW_BUFS, per), np.int8)
    sc = DeviceBuffer((FW_BUFS, FW_ROWS), np.float32)

    def fused(i, store):
        b = i % FW_BUFS
        call("ouro_fwht_rows", src.ptr + 2 * b * per, DT_BF16, dst.ptr + 2 * b * per if store else None, DT_BF16,
             FW_ROWS, FW_N, FW_N, None, 0, xq.ptr + b * per, sc.ptr + 4 * b * FW_ROWS, stream)

    ms_q = time_events(stream, lambda i: fused(i, False), max(steps, 2 * FW_BUFS), warmup)
    ms_qs = time_events(stream, lambda i: fused(i, True), max(steps, 2 * FW_BUFS), warmup)

    # the floor of a call this size: a device-to-device copy of the same
    # 4 MiB of rows (8 MiB moved) over the same rotating buffers
    def copy(i):
        b = i % FW_BUFS
        call("ouro_memcpy_dtod", dst.ptr + 2 * b * per, src.ptr + 2 * b * per, 2 * per, stream)

    ms_cp = time_events(stream, copy, max(steps, 2 * FW_BUFS), warmup)
    return ms, ms_all, ms_q, ms_qs, ms_cp


def bench_prefill(stream, steps, warmup):
    from ouroboros_amd import quant, qwen35
    from ouroboros_amd._lib import GDN_L2NORM_QK, GDN_SCALE_Q, call
    from ouroboros_amd.device import DeviceBuffer

    rng = np.random.default_rng(11)
    T, Hk, Hv, d = PF_T, GDN_HK, GDN_HV, GDN_D
    q = DeviceBuffer.from_host(quant.f32_to_bf16_bits(rng.standard_normal((T, Hk, d)).astype(np.float32)))
    k = DeviceBuffer.from_host(quant.f32_to_bf16_bits(rng.standard_normal((T, Hk, d)).astype(np.float32)))
    v = DeviceBuffer.from_host(quant.f32_to_bf16_bits(rng.standard_normal((T, Hv, d)).astype(np.float32)))
    beta = DeviceBuffer.from_host((1 / (1 + np.exp(-rng.standard_normal((T, Hv))))).astype(np.float32))
    gate = DeviceBuffer.from_host((-np.log1p(np.exp(rng.standard_normal((T, Hv))))).astype(np.float32))
    state = DeviceBuffer.from_host((0.02 * rng.standard_normal((PF_SEQ, Hv, d * d))).astype(np.float32))
    out = DeviceBuffer((T, Hv, d), np.float32)
    cu = np.arange(PF_SEQ + 1, dtype=np.int32) * PF_LEN
    ws = DeviceBuffer((qwen35.chunk_workspace_bytes(T, PF_SEQ, Hv, d, PF_C),), np.uint8)

    def step(_i):
        call("ouro_gdn_chunk_prefill", state.ptr, q.ptr, k.ptr, v.ptr, gate.ptr, beta.ptr, out.ptr,
             cu.ctypes.data, PF_SEQ, T, Hk, Hv, d, PF_C, GDN_L2NORM_QK | GDN_SCALE_Q, 1e-6, ws.ptr, stream)

    return time_events(stream, step, max(3, steps // 5), 2)


# Hybrid stack: 64 prompts of 16..2048 tokens packed varlen, then 128
# greedy decode steps of all 64 sequences (24 layers, 3 delta : 1 attention).
ST_SEQS, ST_MIN, ST_MAX, ST_STEPS = 64, 16, 2048, 128


def stack_lens() -> np.ndarray:
    return np.random.default_rng(5).integers(ST_MIN, ST_MAX + 1, ST_SEQS)


def stack_algorithmic(card, lens) -> dict:
    """Algorithmic HBM bytes of one decode step (every weight byte once,
    delta-net state read + written, the KV cache of every attention layer
    read once, averaged over the steps) and int8 ops of the prefill's
    ternary products (2 x rows x weights, lm_head on the last rows only)."""
    E, F, V, L = card.n_embd, card.n_ff, card.n_vocab, card.n_layer
    d = card.head_dim
    di, dv = card.ssm_n_k_heads * d, card.ssm_n_v_heads * d
    qdim, kvdim = card.n_head * d, card.n_head_kv * d
    n_attn = L // card.full_attention_interval
    n_delta = L - n_attn
    ffn = 3 * E * F
    w_delta = (2 * di + dv) * E + dv * E + 2 * card.ssm_n_v_heads * E + E * dv
    w_attn = 2 * qdim * E + 2 * kvdim * E + E * qdim
    weights = n_delta * (w_delta + ffn) + n_attn * (w_attn + ffn)
    B = len(lens)
    state = n_delta * B * card.ssm_n_v_heads * d * d * 4 * 2
    mean_ctx = float(np.mean(lens)) + (ST_STEPS + 1) / 2
    kv = n_attn * B * mean_ctx * kvdim * 4 * 2
    dec_bytes = weights // 4 + V * E // 4 + state + kv + B * E * 4
    T = int(np.sum(lens))
    pf_ops = 2 * T * weights + 2 * B * V * E
    return {"decode_step_bytes": int(dec_bytes), "weight_bytes": int(weights // 4 + V * E // 4),
            "state_bytes": int(state), "kv_bytes": int(kv), "prefill_int8_ops": int(pf_ops)}


def bench_stack(stream, steps, warmup):
    """One step = a packed prefill of the 64 prompts + 128 decode steps, the
    greedy tokens fed back on the device.  Returns (prefill ms, decode ms
    for all steps, device bytes, prompt tokens)."""
    from ouroboros_amd.device import DeviceBuffer, Event, synchronize
    from ouroboros_amd._lib import call
    from ouroboros_amd.stack import Card, Stack

    card = Card()
    lens = stack_lens()
    T = int(lens.sum())
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    rng = np.random.default_rng(6)
    # the KV pool holds exactly what the run needs: 64-token pages per sequence
    pages = int(sum((int(l) + ST_STEPS + 63) // 64 for l in lens))
    st = Stack(card, 1234, max_seqs=ST_SEQS, max_tokens=T, max_ctx=ST_MAX + ST_STEPS + 1, kv_pages=pages)
    toks = DeviceBuffer.from_host(rng.integers(0, card.n_vocab, T).astype(np.int32))
    a, b = DeviceBuffer((ST_SEQS,), np.int32), DeviceBuffer((ST_SEQS,), np.int32)
    try:
        def run():
            e0, e1, e2 = Event(), Event(), Event()
            e0.record(stream)
            st.prefill(toks, cu, a, None, stream)
            e1.record(stream)
            cur, nxt = a, b
            for _ in range(ST_STEPS):
                st.decode(cur, nxt, None, stream)
                cur, nxt = nxt, cur
            e2.record(stream)
            call("ouro_device_synchronize")
            return e0.elapsed_ms(e1), e1.elapsed_ms(e2)

        for _ in range(max(1, min(warmup, 2))):
            run()
        synchronize(stream)
        pf, dec = [], []
        for _ in range(max(1, min(steps, 3))):
            p, d_ = run()
            pf.append(p)
            dec.append(d_)
        check = stack_check(st, toks, cu, card.n_vocab, stream)
        return float(np.mean(pf)), float(np.mean(dec)), st.device_bytes, T, card, lens, check
    finally:
        st.free()


def stack_check(st, toks, cu, V, stream) -> dict:
    """Untimed sanity check of the benchmark's own workload: one more prefill
    and decode steps with the logits kept; every logit finite and every greedy
    token the first index of its row's largest logit (finite_argmax,
    infer/mod.rs:70-83)."""
    from ouroboros_amd.device import DeviceBuffer, synchronize

    N = len(cu) - 1
    lg = DeviceBuffer((N * V,), np.float32)
    a, b = DeviceBuffer((N,), np.int32), DeviceBuffer((N,), np.int32)
    res = {"finite": True, "tokens_are_argmax": True}
    st.prefill(toks, cu, a, lg, stream)
    for step in range(3):
        if step:
            st.decode(b, a, lg, stream)  # the previous step's tokens in b
        synchronize(stream)
        logits, tok = lg.download().reshape(N, V), a.download()
        res["finite"] &= bool(np.isfinite(logits).all())
        res["tokens_are_argmax"] &= bool(np.array_equal(tok, logits.argmax(axis=1)))
        a, b = b, a
    if not (res["finite"] and res["tokens_are_argmax"]):
        raise SystemExit(f"hybrid stack check failed: {res}")
    return res


COPY_BYTES = 512 << 20


def bench_copy(stream, steps):
    """Device-to-device copy of 512 MiB: the achievable-bandwidth reference
    and the calibration kernel for the FETCH_SIZE / WRITE_SIZE counters."""
    from ouroboros_amd._lib import call
    from ouroboros_amd.device import DeviceBuffer

    src = DeviceBuffer((COPY_BYTES,), np.uint8, zero=True)
    dst = DeviceBuffer((COPY_BYTES,), np.uint8)

    def step(_i):
        call("ouro_memcpy_dtod", dst.ptr, src.ptr, COPY_BYTES, stream)

    return time_events(stream, step, max(3, steps // 5), 2)


def cpu_baseline(orc) -> dict:
    """The reference's own CPU GEMV (matvec_tl1, SSE4.1 order, row-split
    threads, ops.rs:294-321) on the same 6912x2560 shape in its PTQ1_0 form,
    and the bitnet.cpp I2_S / I8_S oracle on the headline format itself."""
    nt, info = cpu_threads()
    rng = np.random.default_rng(5)
    rb = GEMV_IN // 128 * 28
    payload = rng.integers(0, 256, GEMV_OUT * rb, dtype=np.uint8)
    g = payload.reshape(-1, 28)
    d = rng.uniform(0.01, 0.1, g.shape[0]).astype(np.float16).view(np.uint16)
    g[:, 26], g[:, 27] = d & 0xFF, d >> 8
    x = rng.standard_normal(GEMV_IN).astype(np.float32)
    dt, n = cpu_median(lambda: orc.matvec_tl1(payload, GEMV_OUT, GEMV_IN, x, simd=1, nthreads=nt))
    tl1_bytes = payload.nbytes + GEMV_IN * 4 + GEMV_OUT * 4
    i2s = orc.i2s_pack(rng.integers(-1, 2, size=(GEMV_OUT, GEMV_IN)).astype(np.int8), 1.0)

    def i2s_call():
        xq, s = orc.act_quant_i8(x[None])
        orc.gemm_i2s(i2s, GEMV_OUT, GEMV_IN, xq, s, nthreads=nt)

    dt_i2, m = cpu_median(i2s_call, min_runs=10, budget_s=2.0)
    return {
        "value": round(tl1_bytes / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": nt,
        "kind": "port",
        "sample": (f"median of {n} calls (after 3 warm-ups) of the oracle's matvec_tl1 (SSE4.1 lane order, {nt} "
                   f"row-split threads) on one 6912x2560 PTQ1_0 matrix ({tl1_bytes} B per call): "
                   f"{dt * 1e3:.3f} ms/call.  The bitnet.cpp I2_S/I8_S oracle (scalar C, quantisation included) on "
                   f"the headline format: {GEMV_BYTES / dt_i2 / 1e9:.3f} GB/s ({dt_i2 * 1e3:.2f} ms/call, median of "
                   f"{m})"),
        "i2s_oracle_GBs": round(GEMV_BYTES / dt_i2 / 1e9, 3),
        "cpu": _cpu_model(), "threads": info,
    }


def _cpu_model() -> str:
    """/proc/cpuinfo's model name with family / model / stepping, which still
    identify the part where a virtualised host shortens the name."""
    f = {}
    try:
        for line in open("/proc/cpuinfo"):
            if not line.strip():
                break  # the first logical CPU's block
            k, _, v = line.partition(":")
            f[k.strip()] = v.strip()
    except OSError:
        return "unknown"
    ids = ", ".join(f"{k} {f[k]}" for k in ("cpu family", "model", "stepping") if k in f)
    return f"{f.get('model name', 'unknown')} ({ids})" if ids else f.get("model name", "unknown")


def gdn_cpu_baseline(orc) -> dict:
    """delta_head_dim (qwen35.rs:27-57) per (sequence, head), threaded over
    the 32 x 32 heads, on the decode workload."""
    nt, info = cpu_threads()
    rng = np.random.default_rng(3)
    B, Hk, Hv, d = GDN_B, GDN_HK, GDN_HV, GDN_D
    state = (0.02 * rng.standard_normal((B, Hv, d * d))).astype(np.float32)
    q = rng.standard_normal((B, Hk, d)).astype(np.float32)
    k = rng.standard_normal((B, Hk, d)).astype(np.float32)
    v = rng.standard_normal((B, Hv, d)).astype(np.float32)
    gate = -np.log1p(np.exp(rng.standard_normal((B, Hv)))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((B, Hv))))).astype(np.float32)
    dt, n = cpu_median(lambda: orc.gdn_decode(state, q, k, v, gate, beta, B, Hk, Hv, d,
                                              orc.L2NORM_QK | orc.SCALE_Q, 1e-6, nt), budget_s=3.0)
    return {"value": round(B / dt, 1), "unit": "tokens/s", "cores": nt, "kind": "port",
            "sample": f"median of {n} decode steps (after 3 warm-ups) of the oracle's delta_head_dim loop over "
                      f"32x32 heads, {nt} threads: {dt * 1e3:.3f} ms/step",
            "cpu": _cpu_model(), "threads": info}


def fwht_cpu_baseline(orc) -> dict:
    """rotate_fwd (hadamard.rs:41-53) on each of the 512 rows of 4096 (f32,
    as the reference computes), rows over threads; GB/s counts the GPU row's
    bf16 bytes."""
    from ouroboros_amd import quant

    nt, info = cpu_threads()
    rng = np.random.default_rng(7)
    x = rng.standard_normal((FW_ROWS, FW_N)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 50.0
    base = quant.bf16_bits_to_f32(quant.f32_to_bf16_bits(x))
    work = base.copy()

    def call():
        work[:] = base
        orc.rotate_rows(work, None, FW_N, nthreads=nt)

    dt, n = cpu_median(call, budget_s=2.0)
    return {"value": round(FW_BYTES / dt / 1e9, 3), "unit": "GB/s", "cores": nt, "kind": "port",
            "sample": f"median of {n} calls (after 3 warm-ups) of the oracle's rotate_fwd over 512 rows of 4096 "
                      f"(f32, {nt} threads over rows, the copy-in of the input included): {dt * 1e3:.3f} ms/call",
            "cpu": _cpu_model(), "threads": info}


def prefill_cpu_baseline(orc) -> dict:
    """The reference's prefill: each of the 4 sequences token by token through
    delta_head_dim (shell/src/bonsai.rs:48-52 driving qwen35.rs:27-57),
    (sequence, head) pairs over threads, on the 4 x 4096-token workload."""
    nt, info = cpu_threads()
    rng = np.random.default_rng(11)
    # the whole workload: 4 sequences of 4096 tokens (~0.6 s a run on 16 threads)
    L = PF_LEN
    T, Hk, Hv, d = PF_SEQ * L, GDN_HK, GDN_HV, GDN_D
    q = rng.standard_normal((T, Hk, d)).astype(np.float32)
    k = rng.standard_normal((T, Hk, d)).astype(np.float32)
    v = rng.standard_normal((T, Hv, d)).astype(np.float32)
    gate = -np.log1p(np.exp(rng.standard_normal((T, Hv)))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, Hv))))).astype(np.float32)
    state0 = (0.02 * rng.standard_normal((PF_SEQ, Hv, d * d))).astype(np.float32)
    cu = np.arange(PF_SEQ + 1, dtype=np.int32) * L
    st = state0.copy()

    def call():
        st[:] = state0
        orc.gdn_prefill_varlen(st, q, k, v, gate, beta, cu, Hk, Hv, d, orc.L2NORM_QK | orc.SCALE_Q, 1e-6, nt)

    dt, n = cpu_median(call, warmup=1, min_runs=5, budget_s=0.0)
    return {"value": round(T / dt, 1), "unit": "tokens/s", "cores": nt, "kind": "port",
            "sample": f"median of {n} runs (after 1 warm-up) of the oracle's token-loop prefill of the whole "
                      f"workload, 4 x {L} tokens (f32, {nt} threads over the 128 (sequence, head) pairs): "
                      f"{dt * 1e3:.1f} ms/run",
            "cpu": _cpu_model(), "threads": info}


def load_traffic() -> dict:
    """Calibrated HBM bytes per dispatch from the committed PMC summary
    (profiles/pmc_traffic.json, FETCH_SIZE and WRITE_SIZE runs scaled by a
    512 MiB device copy), keyed by kernel name and grid size."""
    f = ROOT / "profiles" / "pmc_traffic.json"
    try:
        return json.loads(f.read_text()).get("kernels", {})
    except (OSError, ValueError):
        return {}


TRAFFIC_SOURCE = ("profiles/pmc_traffic.json: HBM bytes per dispatch from two rocprofv3 --pmc runs of bench.py "
                  "(FETCH_SIZE, then WRITE_SIZE), each scaled by what the counter reads for the 512 MiB device "
                  "copy of the same run; measured in that profiling run, not in this one")


def traffic_of(traffic: dict, prefix: str, grid: int | None = None):
    best = None
    for name, by_grid in traffic.items():
        if not name.startswith(prefix):
            continue
        for g, b in by_grid.items():
            if grid is None or int(g) == grid:
                best = b if best is None else max(best, b)
    return best


def traffic_sum(traffic: dict, prefixes: list[str]):
    """HBM bytes of one call made of several kernels (None if any is unknown)."""
    parts = [traffic_of(traffic, p) for p in prefixes]
    return None if any(b is None for b in parts) else sum(parts)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-stack", action="store_true",
                    help="skip the hybrid-stack leg (profiling runs of the kernel legs)")
    ap.add_argument("--only", choices=["gemv", "gemm", "gdn", "layer", "tl1", "kquant", "fwht", "prefill", "copy",
                                       "stack"],
                    default=None,
                    help="run one workload (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the library has no multi-GPU path "
              "(the workloads would shard by output rows / heads with no exchange).", file=sys.stderr)
        return 2

    from ouroboros_amd import _lib
    
    _lib.init()
    stream = None  # the null stream: no per-launch gap between back-to-back kernels
    orc = None
    if not args.no_cpu:
        import oracle as orc  # the CPU baseline / parity checker only

    res = {}
    if args.only in (None, "gemv"):
        log(f"GEMV 6912x2560 x {GEMV_MATS} matrices")
        res["gemv"] = bench_gemv(stream, args.steps, args.warmup, orc)
    if args.only in (None, "gdn"):
        log("GDN decode B=32")
        res["gdn"] = bench_gdn(stream, args.steps, args.warmup)
    if args.only in (None, "layer"):
        log("GDN layer block B=32")
        res["layer"] = bench_layer(stream, args.steps, args.warmup)
    if args.only in (None, "tl1"):
        log("TL1 matvec 248320x5120 (lm_head probe)")
        res["tl1"] = bench_tl1(stream, args.steps, args.warmup)
    if args.only in (None, "kquant"):
        log("matvec_q on Q8_0 / Q3_K..Q6_K blocks, 248320x5120 and 6912x2560")
        res["kquant"] = bench_kquant(stream, args.steps, args.warmup)
    if args.only in (None, "gemm"):
        log("ternary GEMM 6912x2560, 4..2048 columns")
        res["gemm"] = bench_gemm(stream, args.steps, args.warmup, orc)
    if args.only in (None, "fwht"):
        log("FWHT 512x4096 bf16")
        res["fwht"] = bench_fwht(stream, args.steps, args.warmup)
    if args.only in (None, "copy"):
        log("device copy 512 MiB")
        res["copy"] = bench_copy(stream, args.steps)
    if args.only in (None, "prefill"):
        log("GDN chunked prefill 4x4096")
        res["prefill"] = bench_prefill(stream, args.steps, args.warmup)
    if args.only in (None, "stack") and not args.no_stack:
        log(f"hybrid stack: {ST_SEQS} prompts of {ST_MIN}..{ST_MAX} tokens + {ST_STEPS} decode steps")
        res["stack"] = bench_stack(stream, args.steps, args.warmup)

    traffic = load_traffic()
    out = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "data": "synthetic",
           "traffic_source": TRAFFIC_SOURCE}
    sec = {}
    if "gemv" in res:
        ms, ms_single, ms_small = res["gemv"]
        bytes_launch = GEMV_BYTES * GEMV_MATS
        gbs = bytes_launch / (ms * 1e-3) / 1e9
        out.update({
            "value": round(gbs, 1), "unit": "GB/s", "ms_per_step": round(ms, 4), "dtype": "int8",
            "config": {"workload": "ternary GEMV 6912x2560, 2-bit weights x int8 absmax activations -> fp32, "
                                   f"{GEMV_MATS} distinct matrices per step (one grouped launch, "
                                   f"{GEMV_BYTES * GEMV_MATS / 1e9:.2f} GB)",
                       "out_len": GEMV_OUT, "in_len": GEMV_IN, "matrices_per_step": GEMV_MATS,
                       "bytes_per_matrix": GEMV_BYTES},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": traffic_of(traffic, "i2_gemv_kernel")},
            "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
            "single_matrix_launch_us": round(ms_single * 1e3, 2),
            "single_matrix_GBs": round(GEMV_BYTES / (ms_single * 1e-3) / 1e9, 1),
            f"grouped_{GEMV_MATS_SMALL}_matrices_GBs": round(GEMV_BYTES * GEMV_MATS_SMALL / (ms_small * 1e-3) / 1e9, 1),
        })
    else:
        out.update({"value": None, "unit": "GB/s"})
    if "gdn" in res:
        ms = res["gdn"]
        gbs = GDN_BYTES / (ms * 1e-3) / 1e9
        sec["gdn_decode"] = {
            "value": round(GDN_B / (ms * 1e-3), 1), "unit": "tokens/s", "ms_per_step": round(ms, 4),
            "config": "B=32 seqs, Hk=16, Hv=32, d=128, fp32 state, bf16 q/k/v, 8 rotating state sets",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_of(traffic, "gdn_decode_kernel")},
            "bytes_per_step": GDN_BYTES,
        }
    if "layer" in res:
        ms = res["layer"]
        gbs = LY_BYTES / (ms * 1e-3) / 1e9
        sec["gdn_layer_block"] = {
            "value": round(GDN_B / (ms * 1e-3), 1), "unit": "tokens/s", "ms_per_step": round(ms, 4),
            "config": "run_delta's block between the projections: gates, conv+SiLU, normed recurrence, gated RMS "
                      "norm, V-grouped; B=32, Hk=16, Hv=32, d=128, f32, 8 rotating state sets (2 launches)",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)},
            "bytes_per_step": LY_BYTES,
        }
    if "tl1" in res:
        ms, ms_am, ms_raw, ms_tq1, tq1_bytes, kcols = res["tl1"]
        gbs = TL1_BYTES / (ms * 1e-3) / 1e9
        sec["tl1_matvec_lmhead"] = {
            "value": round(gbs, 1), "unit": "GB/s", "ms_per_call": round(ms, 4),
            "config": "TL1 (PTQ1_0) 248320x5120 resident weight (table-lookup GEMV), fp32 x and y, the reference's "
                      "lm_head probe payload (ops.rs:694-717; its CPU figure is 1.75 GB/s on an i7-3770)",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_of(traffic, "tl1_lut_kernel", 256000)},
            "bytes_per_call": TL1_BYTES,
            "greedy_sample_ms": round(ms_am, 4),
            "greedy_sample_tokens_per_s": round(1e3 / ms_am, 1),
            "raw_payload_matvec_q_ms": round(ms_raw, 4),
            "raw_payload_matvec_q_GBs": round(TL1_BYTES / (ms_raw * 1e-3) / 1e9, 1),
            "raw_tq1_0_matvec_q_ms": round(ms_tq1, 4),
            "raw_tq1_0_matvec_q_GBs": round((tq1_bytes + 4 * (TL1_IN + TL1_OUT)) / (ms_tq1 * 1e-3) / 1e9, 1),
            "k_columns": {
                "config": "ouro_weight_matmul of a resident TL1 handle (max_cols 8) for K columns: K = 1 the "
                          "table-lookup matvec, K >= 2 one int8 MFMA pass over the trits for all K",
                "by_k": kcols,
                "k8_over_k1": {r0["shape"]: round(r8["us_per_call"] / r0["us_per_call"], 2)
                               for r0 in kcols if r0["k"] == 1 for r8 in kcols
                               if r8["k"] == 8 and r8["shape"] == r0["shape"]},
            },
        }
    if "kquant" in res:
        rows = res["kquant"]
        big = [r for r in rows if r["out_len"] == TL1_OUT]
        kind_id = {name: kind for name, kind, _bb, _be in KQ_KINDS}
        for r in big:  # the lm_head launch of each kind's GEMV
            if r["kind"] == "Q3_K":  # the matrix-core kernels: workgroups of 256 threads, 4 a CU
                r["traffic"] = traffic_of(traffic, "kq3_mfma_kernel<1>", 262144)
            elif r["kind"] in ("Q4_K", "Q5_K"):  # the shared 16-row tiles
                r["traffic"] = traffic_of(traffic, f"kq45_mfma_kernel<{kind_id[r['kind']]}, true>", 262144)
            elif r["kind"] == "Q6_K":  # 3 workgroups a CU
                r["traffic"] = traffic_of(traffic, "kq6_mfma_kernel<14, true>", 196608)
            elif r["kind"] == "Q8_0":
                r["traffic"] = traffic_of(traffic, "kq8_mfma_kernel", 262144)
            else:
                r["traffic"] = traffic_of(traffic, f"kq_gemv_kernel<{kind_id[r['kind']]},", 491520)
        slow = min(big, key=lambda r: r["GBs"])
        sec["kquant_matvec"] = {
            "value": slow["GBs"], "unit": "GB/s",
            "config": "ouro_matvec_q on raw ggml Q8_0 / Q3_K / Q4_K / Q5_K / Q6_K blocks (matvec_qblock, "
                      "ops.rs:101-128), fp32 x and y; value = the slowest kind at 248320x5120",
            "roofline": {"bound": "hbm", "achieved": slow["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": slow["frac"], "traffic": slow["traffic"]},
            "by_kind": rows,
        }
    if "gemm" in res:
        rows, vendor = res["gemm"]
        main = next(r for r in rows if r["cols"] == GM_COLS_MAIN)
        sec["ternary_gemm"] = {
            "value": main["mfma_tops"], "unit": "TOP/s", "us_per_call": main["mfma_us"],
            "config": f"I2 6912x2560 x int8 [{GM_COLS_MAIN} columns] -> fp32, int8 MFMA (the K-column matmul_q)",
            "roofline": {"bound": "mfma", "achieved": main["mfma_tops"], "peak": INT8_MFMA_PEAK_TOPS,
                         "unit": "TOP/s", "frac": round(main["mfma_tops"] / INT8_MFMA_PEAK_TOPS, 4),
                         "traffic": traffic_of(traffic, "i2_gemm_big_kernel")},
            "algorithmic_bytes": GM_OUT * GM_IN // 4 + GM_COLS_MAIN * GM_IN + GM_COLS_MAIN * GM_OUT * 4,
            "by_columns": rows,
            "vendor_int8_gemm_8bit_weights_us": round(vendor * 1e3, 2) if vendor else None,
        }
    if "fwht" in res:
        ms, ms_all, ms_q, ms_qs, ms_cp = res["fwht"]
        gbs = FW_BYTES / (ms * 1e-3) / 1e9
        gbs_all = FW_BYTES * FW_BUFS / (ms_all * 1e-3) / 1e9
        sec["fwht"] = {
            "value": round(gbs, 1), "unit": "GB/s", "ms_per_call": round(ms, 4),
            "config": "512x4096 bf16 in/out, block 4096, scale 1/64, 32 rotating buffers",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_of(traffic, "fwht_row_kernel", FW_ROWS * 256)},
            "streaming_16384_rows_GBs": round(gbs_all, 1),
            "bytes_per_call": FW_BYTES,
            "same_size_copy": {"config": "hipMemcpyAsync device-to-device of the call's 4 MiB of bf16 rows "
                                         "(8 MiB moved), same 32 rotating buffers: the floor of a call this size",
                               "ms_per_call": round(ms_cp, 4),
                               "GBs": round(FW_BYTES / (ms_cp * 1e-3) / 1e9, 1),
                               "frac": round(FW_BYTES / (ms_cp * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
            "fused_int8_epilogue": {
                "config": "the same rotation with each bf16 row quantised to int8 (quantize_row_i8_s) in the "
                          "kernel's epilogue; bf16 rows not stored / stored",
                "bytes_per_call": FW_Q_BYTES, "ms_per_call": round(ms_q, 4),
                "GBs": round(FW_Q_BYTES / (ms_q * 1e-3) / 1e9, 1),
                "frac": round(FW_Q_BYTES / (ms_q * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "with_bf16_store_bytes": FW_Q_BYTES + FW_BYTES // 2, "with_bf16_store_ms": round(ms_qs, 4),
                "with_bf16_store_GBs": round((FW_Q_BYTES + FW_BYTES // 2) / (ms_qs * 1e-3) / 1e9, 1),
            },
        }
    if "copy" in res:
        ms = res["copy"]
        sec["device_copy"] = {"value": round(2 * COPY_BYTES / (ms * 1e-3) / 1e9, 1), "unit": "GB/s",
                              "config": "hipMemcpyAsync device-to-device, 512 MiB (read + write counted)",
                              "frac_of_peak": round(2 * COPY_BYTES / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    if "prefill" in res:
        ms = res["prefill"]
        tf = PF_FLOPS / (ms * 1e-3) / 1e12
        gbs = PF_BYTES / (ms * 1e-3) / 1e9
        t_mem = PF_BYTES / (HBM_PEAK_GBS * 1e9)
        t_mfma = PF_FLOPS / (MFMA_BF16_PEAK_TFLOPS * 1e12)
        sec["gdn_prefill"] = {
            "value": round(PF_T / (ms * 1e-3), 1), "unit": "tokens/s", "ms_per_call": round(ms, 4),
            "config": "4 seqs x 4096 tokens packed varlen, chunk 64, Hk=16, Hv=32, d=128, bf16 q/k/v, fp32 state/out",
            # the binding roof: at 154 flop/B (below the bf16 ridge of 312) HBM bounds the call
            "roofline": {"bound": "hbm" if t_mem >= t_mfma else "mfma", "achieved": round(gbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(max(t_mem, t_mfma) / (ms * 1e-3), 4),
                         "traffic": traffic_sum(traffic, ["gdn_chunk_prep_kernel", "gdn_chunk_scan_kernel"])},
            "mfma_roofline": {"achieved": round(tf, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                              "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)},
            "algorithmic_gflop": round(PF_FLOPS / 1e9, 2), "bytes": PF_BYTES, "hbm_GBs": round(gbs, 1),
        }
    if "stack" in res:
        pf_ms, dec_ms, dev_bytes, T, card, lens, check = res["stack"]
        alg = stack_algorithmic(card, lens)
        step_ms = dec_ms / ST_STEPS
        dec_gbs = alg["decode_step_bytes"] / (step_ms * 1e-3) / 1e9
        pf_tops = alg["prefill_int8_ops"] / (pf_ms * 1e-3) / 1e12
        gen = ST_SEQS * ST_STEPS
        sec["hybrid_stack"] = {
            "value": round((T + gen) / ((pf_ms + dec_ms) * 1e-3), 1), "unit": "tokens/s",
            "ms_per_step": round(pf_ms + dec_ms, 3),
            "config": f"24 layers (18 gated delta-net, 6 full attention), hidden 2560, FFN 6912, vocab 248320, "
                      f"I2 ternary projections on Hadamard-rotated int8 activations; {ST_SEQS} prompts of "
                      f"{ST_MIN}..{ST_MAX} tokens ({T} total) packed varlen, then {ST_STEPS} greedy decode steps "
                      f"of all {ST_SEQS} sequences; synthetic seeded weights",
            "prefill_tokens_per_s": round(T / (pf_ms * 1e-3), 1), "prefill_ms": round(pf_ms, 3),
            "decode_tokens_per_s": round(gen / (dec_ms * 1e-3), 1), "decode_step_ms": round(step_ms, 4),
            "decode_roofline": {"bound": "hbm", "achieved": round(dec_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(dec_gbs / HBM_PEAK_GBS, 4)},
            "prefill_ternary_TOPs": round(pf_tops, 1),
            "algorithmic": alg, "device_bytes": int(dev_bytes),
            "output_check": check,
        }
    if orc is not None:
        log("CPU baselines")
        if "gemv" in res:
            out["cpu_baseline"] = cpu_baseline(orc)
        if "gdn" in res:
            sec.setdefault("gdn_decode", {})["cpu_baseline"] = gdn_cpu_baseline(orc)
        if "fwht" in res:
            sec.setdefault("fwht", {})["cpu_baseline"] = fwht_cpu_baseline(orc)
        if "prefill" in res:
            sec.setdefault("gdn_prefill", {})["cpu_baseline"] = prefill_cpu_baseline(orc)
    out["secondary"] = sec
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

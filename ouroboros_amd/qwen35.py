"""Gated delta-net recurrence on the GPU.

``delta_head_dim`` mirrors cluster/src/infer/qwen35.rs:27-57 (one head, in
place).  ``gdn_decode`` is the batched decode step over sequences and
v-heads with run_delta's per-head preprocessing (qwen35.rs:1096-1112);
``gdn_chunk_prefill`` runs a packed varlen prefill in chunks and equals the
token-by-token recurrence.  ``gdn_layer_decode`` is the whole layer block
of run_delta around the recurrence (gates, conv + SiLU, gated RMS norm;
qwen35.rs:1066-1140).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import call
from .device import DeviceBuffer

S = 128  # d_state of the qwen35 family (qwen35.rs:8)


@dataclass
class DeltaStep:
    """Per-head gate (log-decay) and beta of one step (qwen35.rs:12-15)."""

    gate: float
    beta: float


def delta_q_scale() -> float:
    """q scale of the recurrence (qwen35.rs:108-110)."""
    return float(np.float32(1.0) / np.sqrt(np.float32(S)))


def delta_head_dim(state, sdim: int, q, k, v, step: DeltaStep, out, stream=None) -> None:
    """One recurrence step for one head, in place (qwen35.rs:27)."""
    bufs = []
    for a in (state, q, k, v, out):
        bufs.append(a if isinstance(a, DeviceBuffer) else DeviceBuffer.from_host(
            np.ascontiguousarray(a, dtype=np.float32)))
    sb, qb, kb, vb, ob = bufs
    call("ouro_delta_head_dim", sb.ptr, sdim, qb.ptr, kb.ptr, vb.ptr, float(step.gate),
         float(step.beta), ob.ptr, stream)
    if not isinstance(state, DeviceBuffer):
        state[...] = sb.download().reshape(np.shape(state))
    if not isinstance(out, DeviceBuffer):
        out[...] = ob.download().reshape(np.shape(out))


def _dt(b: DeviceBuffer) -> int:
    return _lib.DT_BF16 if b.dtype == np.uint16 else _lib.DT_F32


def gdn_decode(state: DeviceBuffer, q: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer,
               gate: DeviceBuffer, beta: DeviceBuffer, out: DeviceBuffer, B: int, Hk: int,
               Hv: int, d: int = S, flags: int = _lib.GDN_L2NORM_QK | _lib.GDN_SCALE_Q,
               eps: float = 1e-6, stream=None) -> None:
    if q.dtype != k.dtype:
        raise ValueError("q and k must share a dtype")
    call("ouro_gdn_decode", state.ptr, q.ptr, k.ptr, _dt(q), v.ptr, _dt(v), gate.ptr, beta.ptr,
         out.ptr, B, Hk, Hv, d, flags, eps, stream)


def gdn_chunk_prefill(state: DeviceBuffer, q: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer,
                      gate: DeviceBuffer, beta: DeviceBuffer, out: DeviceBuffer,
                      cu_seqlens: np.ndarray | None, T: int, Hk: int, Hv: int, d: int = S,
                      chunk: int = 64, flags: int = _lib.GDN_L2NORM_QK | _lib.GDN_SCALE_Q,
                      eps: float = 1e-6, workspace: DeviceBuffer | None = None, stream=None) -> None:
    """Chunked prefill of packed varlen sequences (q, k, v bf16 as uint16).

    ``workspace`` (optional) is a device buffer of at least
    ``chunk_workspace_bytes(T, n, Hv)`` bytes; without it the library's
    per-device workspace is used."""
    if cu_seqlens is None:
        cu, n = None, 1
    else:
        cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        n = len(cu) - 1
    call("ouro_gdn_chunk_prefill", state.ptr, q.ptr, k.ptr, v.ptr, gate.ptr, beta.ptr, out.ptr,
         cu.ctypes.data if cu is not None else None, n, T, Hk, Hv, d, chunk, flags, eps,
         workspace.ptr if workspace is not None else None, stream)


def chunk_workspace_bytes(T: int, N: int, Hv: int, d: int = S, chunk: int = 64) -> int:
    """Bytes of the per-chunk records gdn_chunk_prefill writes (0 = unsupported shape)."""
    return int(_lib.lib().ouro_gdn_chunk_workspace_bytes(T, N, Hv, d, chunk))


def layer_workspace_bytes(B: int, Hk: int, Hv: int, d: int = S) -> int:
    """Bytes of scratch gdn_layer_decode uses: 0 (one launch, no scratch)."""
    return int(_lib.lib().ouro_gdn_layer_workspace_bytes(B, Hk, Hv, d))


def gdn_layer_decode(qkv: DeviceBuffer, z: DeviceBuffer, beta_raw: DeviceBuffer, alpha_raw: DeviceBuffer,
                     dt_bias: DeviceBuffer, a_log: DeviceBuffer, conv_w: DeviceBuffer, norm_w: DeviceBuffer,
                     conv_state: DeviceBuffer, state: DeviceBuffer, out: DeviceBuffer, B: int, Hk: int, Hv: int,
                     d: int = S, flags: int = 0, eps: float = 1e-6, workspace: DeviceBuffer | None = None,
                     stream=None) -> None:
    """The delta-net layer block of one decode step (run_delta, qwen35.rs:1066-1140):
    gates, conv + SiLU, normed recurrence and gated RMS norm for B sequences.
    conv_state and state are updated in place; all buffers f32."""
    call("ouro_gdn_layer_decode", qkv.ptr, z.ptr, beta_raw.ptr, alpha_raw.ptr, dt_bias.ptr, a_log.ptr,
         conv_w.ptr, norm_w.ptr, conv_state.ptr, state.ptr, out.ptr, B, Hk, Hv, d, flags, eps,
         workspace.ptr if workspace is not None else None, stream)

"""Ternary / quantised matvec and matmul on the GPU.

``matvec_q`` and ``matmul_q`` mirror the reference kernel-call surface
(cluster/src/infer/ops.rs:76-84 and 219-230): y = W x for a payload of a
given kind, with matmul's output column-major ``y[c*out_len + r]``.  Host
numpy arguments are uploaded per call (the reference takes host slices);
for resident weights use :class:`Weight`, the device analogue of the
reference's GpuPool (ouro-wgpu/src/lib.rs:251-356).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import call
from .device import DeviceBuffer
from .quant import QuantKind


def _dev(a, dtype) -> tuple[DeviceBuffer, bool]:
    if isinstance(a, DeviceBuffer):
        return a, False
    return DeviceBuffer.from_host(np.ascontiguousarray(a, dtype=dtype)), True


def matvec_q(payload, kind, out_len: int, in_len: int, x, stream=None):
    """y = W x (ops.rs:76).  Returns numpy when x is numpy, else a DeviceBuffer."""
    return matmul_q(payload, kind, out_len, in_len, x, 1, stream)


def matmul_q(payload, kind, out_len: int, in_len: int, x, k: int, stream=None):
    """y = W X for k row-major input columns; y column-major [k*out_len] (ops.rs:219)."""
    host_out = not isinstance(x, DeviceBuffer)
    pb, _ = _dev(payload, np.uint8)
    xb, _ = _dev(x, np.float32)
    y = DeviceBuffer((k * out_len,), np.float32)
    call("ouro_matmul_q", pb.ptr, int(kind), out_len, in_len, xb.ptr, k, y.ptr, stream)
    return y.download() if host_out else y


def i2_tiled_bytes(out_len: int, in_len: int) -> int:
    return int(_lib.lib().ouro_i2_tiled_bytes(out_len, in_len))


def i2_payload(canonical: np.ndarray | DeviceBuffer, out_len: int, in_len: int, w_scale: float,
               stream=None) -> DeviceBuffer:
    """Device OURO_KIND_I2 payload (tiled codes + fp32 scale) from canonical bytes."""
    cb, _ = _dev(canonical, np.uint8)
    tb = i2_tiled_bytes(out_len, in_len)
    if tb == 0:
        raise ValueError(f"I2 needs in_len % 256 == 0 (got {in_len})")
    out = DeviceBuffer((tb + 16,), np.uint8)
    sc = DeviceBuffer.from_host(np.array([w_scale], dtype=np.float32))
    call("ouro_i2_tile", cb.ptr, out_len, in_len, out.ptr, sc.ptr, stream)
    return out


def i2s_payload(i2s: np.ndarray | DeviceBuffer, out_len: int, in_len: int, stream=None) -> DeviceBuffer:
    """Device OURO_KIND_I2 payload (tiled codes + the tensor's scale) from a bitnet.cpp I2_S tensor."""
    ib, _ = _dev(i2s, np.uint8)
    tb = i2_tiled_bytes(out_len, in_len)
    if tb == 0:
        raise ValueError(f"I2_S repack needs in_len % 256 == 0 (got {in_len})")
    out = DeviceBuffer((tb + 16,), np.uint8)
    call("ouro_i2s_tile", ib.ptr, out_len, in_len, out.ptr, stream)
    return out


def i2s_mfma_payload(i2s: np.ndarray | DeviceBuffer, out_len: int, in_len: int, stream=None) -> DeviceBuffer:
    """Device MFMA-tiled codes + the tensor's scale from a bitnet.cpp I2_S tensor."""
    ib, _ = _dev(i2s, np.uint8)
    tb = i2_mfma_bytes(out_len, in_len)
    if tb == 0:
        raise ValueError(f"I2_S repack needs in_len % 256 == 0 (got {in_len})")
    out = DeviceBuffer((tb + 16,), np.uint8)
    call("ouro_i2s_tile_mfma", ib.ptr, out_len, in_len, out.ptr, stream)
    return out


def i2_mfma_bytes(out_len: int, in_len: int) -> int:
    return int(_lib.lib().ouro_i2_mfma_bytes(out_len, in_len))


def i2_mfma_payload(canonical: np.ndarray | DeviceBuffer, out_len: int, in_len: int, w_scale: float,
                    stream=None) -> DeviceBuffer:
    """Device MFMA-tiled I2 codes + fp32 scale (for gemm_i2_mfma) from canonical bytes."""
    cb, _ = _dev(canonical, np.uint8)
    tb = i2_mfma_bytes(out_len, in_len)
    if tb == 0:
        raise ValueError(f"I2 needs in_len % 256 == 0 (got {in_len})")
    out = DeviceBuffer((tb + 16,), np.uint8)
    sc = DeviceBuffer.from_host(np.array([w_scale], dtype=np.float32))
    call("ouro_i2_tile_mfma", cb.ptr, out_len, in_len, out.ptr, sc.ptr, stream)
    return out


def gemm_i2_mfma(w_payload: DeviceBuffer, out_len: int, in_len: int, xq: DeviceBuffer,
                 act_scale: DeviceBuffer, ncols: int, y: DeviceBuffer, acc: DeviceBuffer | None = None,
                 stream=None) -> None:
    """MFMA-tiled I2 x int8 columns -> fp32 (and optionally the exact int32 sums)."""
    tb = i2_mfma_bytes(out_len, in_len)
    call("ouro_gemm_i2_mfma", w_payload.ptr, out_len, in_len, w_payload.ptr + tb, xq.ptr, act_scale.ptr,
         ncols, y.ptr, acc.ptr if acc is not None else None, stream)


def act_quant_i8(x: DeviceBuffer, rows: int, n: int, xq: DeviceBuffer, act_scale: DeviceBuffer,
                 stream=None) -> None:
    """quantize_row_i8_s (bitnet.cpp) per row: int8 rows and act_scale = 127 / max(amax, 1e-5)."""
    dt = _lib.DT_BF16 if x.dtype == np.uint16 else _lib.DT_F32
    call("ouro_act_quant_i8", x.ptr, dt, rows, n, xq.ptr, act_scale.ptr, stream)


def gemm_i2(w_payload: DeviceBuffer, out_len: int, in_len: int, xq: DeviceBuffer,
            act_scale: DeviceBuffer, ncols: int, y: DeviceBuffer, acc: DeviceBuffer | None = None,
            stream=None) -> None:
    """Tiled-I2 x int8 columns -> fp32 (and optionally the exact int32 sums)."""
    tb = i2_tiled_bytes(out_len, in_len)
    call("ouro_gemm_i2", w_payload.ptr, out_len, in_len, w_payload.ptr + tb, xq.ptr, act_scale.ptr,
         ncols, y.ptr, acc.ptr if acc is not None else None, stream)


class Weight:
    """A resident weight handle (GpuPool::upload_q6k / matvec pattern)."""

    def __init__(self, kind, host_payload: np.ndarray, out_len: int, in_len: int,
                 w_scale: float = 1.0, max_cols: int = 8):
        _lib.init()
        self.kind = QuantKind(kind)
        self.out_len, self.in_len = out_len, in_len
        arr = np.ascontiguousarray(host_payload, dtype=np.uint8)
        h = C.c_void_p()
        call("ouro_weight_upload", int(kind), arr.ctypes.data, arr.nbytes, out_len, in_len,
             float(w_scale), max_cols, C.byref(h))
        self.handle = h.value

    def matvec(self, x, stream=None):
        return self.matmul(x, 1, stream)

    def matmul(self, x, k: int, stream=None):
        host_out = not isinstance(x, DeviceBuffer)
        xb, _ = _dev(x, np.float32)
        y = DeviceBuffer((k * self.out_len,), np.float32)
        call("ouro_weight_matmul", self.handle, xb.ptr, k, y.ptr, stream)
        return y.download() if host_out else y

    def matvec_argmax(self, x, y: DeviceBuffer | None = None, stream=None) -> int:
        """finite_argmax(W x) (Qwen35Stage::sample, qwen35.rs:746-757); y optionally keeps the logits."""
        xb, _ = _dev(x, np.float32)
        idx = DeviceBuffer((1,), np.int32)
        call("ouro_weight_matvec_argmax", self.handle, xb.ptr, y.ptr if y is not None else None, idx.ptr, stream)
        return int(idx.download()[0])

    def free(self) -> None:
        if self.handle is not None:
            call("ouro_weight_free", self.handle)
            self.handle = None

    def __del__(self):
        try:
            if getattr(self, "handle", None) is not None and _lib._LIB is not None:
                _lib.lib().ouro_weight_free(self.handle)
                self.handle = None
        except Exception:
            pass


def finite_argmax(y) -> int:
    """finite_argmax (infer/mod.rs:70-83) of a device (or host) float vector, on the GPU."""
    yb, _ = _dev(y, np.float32)
    idx = DeviceBuffer((1,), np.int32)
    call("ouro_finite_argmax", yb.ptr, yb.nbytes // yb.dtype.itemsize, idx.ptr, None)
    return int(idx.download()[0])

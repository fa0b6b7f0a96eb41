"""Walsh-Hadamard activation rotation on the GPU.

``rotate_fwd`` / ``rotate_inv`` mirror cluster/src/infer/hadamard.rs:41-66
(in place on an fp32 vector, signs of the same length, power-of-two block);
``fwht_rows`` is the row-batched form with bf16 I/O and the fused int8
absmax epilogue.  The fp32 results are bit-identical to the reference.
"""
from __future__ import annotations

import numpy as np

from . import _lib
from ._lib import call
from .device import DeviceBuffer


def _rotate(name: str, x, signs, block_size: int, stream=None) -> None:
    host = not isinstance(x, DeviceBuffer)
    xb = DeviceBuffer.from_host(np.ascontiguousarray(x, dtype=np.float32)) if host else x
    sb = signs if isinstance(signs, DeviceBuffer) else DeviceBuffer.from_host(
        np.ascontiguousarray(signs, dtype=np.float32))
    n = int(np.prod(xb.shape))
    if int(np.prod(sb.shape)) != n:
        raise _lib.OuroError(name, 1, "sign vector must match activation")
    call(name, xb.ptr, sb.ptr, n, block_size, stream)
    if host:
        x[...] = xb.download().reshape(np.shape(x))


def rotate_fwd(x, signs, block_size: int, stream=None) -> None:
    """x' = H (s o x) / sqrt(N), blockwise, in place (hadamard.rs:41)."""
    _rotate("ouro_rotate_fwd", x, signs, block_size, stream)


def rotate_inv(x, signs, block_size: int, stream=None) -> None:
    """h = s o (H z) / sqrt(N), blockwise, in place (hadamard.rs:57)."""
    _rotate("ouro_rotate_inv", x, signs, block_size, stream)


def fwht_rows(x: DeviceBuffer, y: DeviceBuffer | None, rows: int, n: int, block: int,
              signs: DeviceBuffer | None = None, inverse: bool = False,
              xq: DeviceBuffer | None = None, act_scale: DeviceBuffer | None = None,
              stream=None) -> None:
    """Rotate `rows` rows of n (dtype from the buffers: float32 or bf16 as uint16)."""
    dt = lambda b: _lib.DT_BF16 if b.dtype == np.uint16 else _lib.DT_F32
    call("ouro_fwht_rows", x.ptr, dt(x), y.ptr if y is not None else None,
         dt(y) if y is not None else _lib.DT_F32, rows, n, block,
         signs.ptr if signs is not None else None, _lib.FWHT_INVERSE if inverse else 0,
         xq.ptr if xq is not None else None, act_scale.ptr if act_scale is not None else None, stream)

"""Quant kinds and the 2-bit ternary packings (host side, no GPU needed).

``QuantKind`` mirrors the reference enum (cluster/src/infer/dequant.rs:315-388)
with the same ggml dtype ids.  ``I2_S`` is bitnet.cpp's 2-bit ternary tensor
(GGML_TYPE_I2_S of microsoft/BitNet's ggml fork, the reference's bitnet-cpp
submodule); ``I2`` is this library's resident (device-tiled) layout of the
same codes.
"""
from __future__ import annotations

import enum

import numpy as np

from . import _lib


class QuantKind(enum.IntEnum):
    F32 = _lib.KIND_F32
    F16 = _lib.KIND_F16
    BF16 = _lib.KIND_BF16
    Q8_0 = _lib.KIND_Q8_0
    Q3K = _lib.KIND_Q3K
    Q4K = _lib.KIND_Q4K
    Q5K = _lib.KIND_Q5K
    Q6K = _lib.KIND_Q6K
    TQ1_0 = _lib.KIND_TQ1_0
    TL1 = _lib.KIND_TL1
    I2_S = _lib.KIND_I2_S
    I2 = _lib.KIND_I2

    @classmethod
    def from_dtype(cls, dtype_id: int) -> "QuantKind | None":
        """QuantKind::from_dtype (dequant.rs:334-348): the reference's set of
        ggml dtype ids; None for any other id, I2_S's 36 included (bitnet.cpp
        tensors are uploaded by kind, not from a shard's dtype)."""
        try:
            k = cls(dtype_id)
        except ValueError:
            return None
        return None if k in (cls.I2, cls.I2_S) else k

    def block_bytes(self) -> int:  # dequant.rs:351-363
        return {self.F32: 4, self.F16: 2, self.BF16: 2, self.TQ1_0: 54, self.TL1: 28, self.I2_S: 32,
                self.I2: 1, self.Q8_0: 34, self.Q3K: 110, self.Q4K: 144, self.Q5K: 176, self.Q6K: 210}[self]

    def block_elems(self) -> int:  # dequant.rs:366-373
        return {self.F32: 1, self.F16: 1, self.BF16: 1, self.TQ1_0: 256, self.TL1: 128, self.I2_S: 128,
                self.I2: 4, self.Q8_0: 32, self.Q3K: 256, self.Q4K: 256, self.Q5K: 256, self.Q6K: 256}[self]

    def row_bytes(self, k: int) -> int:  # dequant.rs:376-387
        return k // self.block_elems() * self.block_bytes()


def i2_pack(w: np.ndarray) -> np.ndarray:
    """Canonical I2 bytes of a ternary matrix w[out][in] (values -1, 0, +1).

    Weight k of a row sits in byte k/4 at bits 2*(k%4) as code w+1.
    """
    w = np.asarray(w)
    if w.ndim != 2 or w.shape[1] % 4:
        raise ValueError("i2_pack: need a 2-D matrix with in_len % 4 == 0")
    if w.size and (w.min() < -1 or w.max() > 1):
        raise ValueError("i2_pack: weights must be in {-1, 0, +1}")
    codes = (w.astype(np.int16) + 1).astype(np.uint8).reshape(w.shape[0], -1, 4)
    return (codes[..., 0] | (codes[..., 1] << 2) | (codes[..., 2] << 4) | (codes[..., 3] << 6)).astype(np.uint8)


def i2_unpack(packed: np.ndarray, in_len: int) -> np.ndarray:
    """Inverse of :func:`i2_pack` (code 3 decodes to +2)."""
    p = np.asarray(packed, dtype=np.uint8).reshape(-1, in_len // 4)
    codes = np.stack([(p >> (2 * f)) & 3 for f in range(4)], axis=-1).reshape(p.shape[0], in_len)
    return codes.astype(np.int8) - 1


def i2s_pack(w: np.ndarray, w_scale: float) -> np.ndarray:
    """bitnet.cpp I2_S bytes of ternary w[out][in] with per-tensor scale w_scale > 0.

    These are the bytes quantize_i2_s makes of w * w_scale: the flattened
    weights go in blocks of 128; weight j of block b sits in byte
    32*b + j%32 at bits 6 - 2*(j/32) as code w+1; the fp32 scale
    max|w * w_scale| (w_scale, or 0 for an all-zero w) follows the n/4 code
    bytes, then 28 zero bytes (quantize_i2_s writes n/4 + 32 bytes).
    """
    w = np.asarray(w)
    if w.ndim != 2 or w.size % 128:
        raise ValueError("i2s_pack: need a 2-D matrix with a multiple of 128 elements")
    if w.size and (w.min() < -1 or w.max() > 1):
        raise ValueError("i2s_pack: weights must be in {-1, 0, +1}")
    if not w_scale > 0:
        raise ValueError("i2s_pack: w_scale must be positive")
    codes = (w.astype(np.int16) + 1).astype(np.uint8).reshape(-1, 4, 32)  # [block][j/32][j%32]
    packed = (codes[:, 0] << 6) | (codes[:, 1] << 4) | (codes[:, 2] << 2) | codes[:, 3]
    out = np.zeros(w.size // 4 + 32, np.uint8)
    out[: w.size // 4] = packed.reshape(-1)
    scale = np.float32(w_scale) if w.any() else np.float32(0.0)
    out[w.size // 4: w.size // 4 + 4] = np.array([scale], np.float32).view(np.uint8)
    return out


def i2s_unpack(buf: np.ndarray, out_len: int, in_len: int) -> tuple[np.ndarray, float]:
    """Inverse of :func:`i2s_pack`: (w[out][in] with code 3 as +2, the fp32 scale)."""
    b = np.asarray(buf, dtype=np.uint8)
    n = out_len * in_len
    p = b[: n // 4].reshape(-1, 32)
    codes = np.stack([(p >> (6 - 2 * f)) & 3 for f in range(4)], axis=1)  # [block][j/32][j%32]
    scale = float(b[n // 4: n // 4 + 4].view(np.float32)[0])
    return codes.reshape(out_len, in_len).astype(np.int8) - 1, scale


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x7FFFFF) != 0)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> fp32 (exact; dequant.rs:197-199)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)

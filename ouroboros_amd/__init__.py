"""ouroboros_amd: MI355X (gfx950) kernels for OuroborOS's quantized-inference
hot path behind a C ABI (include/ouro_hip.h).

Modules: ``ops`` (ternary / quantised matvec and matmul), ``hadamard``
(Walsh-Hadamard rotation), ``qwen35`` (gated delta-net decode and chunked
prefill), ``quant`` (kinds and I2 packing), ``device`` (buffers, streams,
events).  The compute runs only in libouro_hip.so; there is no CPU fallback.
"""
from ._lib import OuroError, gpu_available, init, lib  # noqa: F401

__all__ = ["OuroError", "gpu_available", "init", "lib"]

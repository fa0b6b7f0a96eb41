"""Hybrid decoder stack (include/ouro_stack.h) from Python: the reference's
Qwen35Stage forward / sample (cluster/src/infer/qwen35.rs:730-805) for a
continuous batch of sequences, with synthetic weights generated from a seed.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import StackCard, call
from .device import DeviceBuffer


@dataclass
class Card:
    n_layer: int = 24
    n_embd: int = 2560
    n_ff: int = 6912
    n_vocab: int = 248320
    full_attention_interval: int = 4
    n_head: int = 16
    n_head_kv: int = 4
    head_dim: int = 128
    n_rot: int = 64
    ssm_n_k_heads: int = 16
    ssm_n_v_heads: int = 32
    ssm_d_state: int = 128
    eps: float = 1e-6
    rope_base: float = 1e7

    def c(self) -> StackCard:
        return StackCard(**{k: getattr(self, k) for k, _ in StackCard._fields_})


class Stack:
    def __init__(self, card: Card, seed: int, max_seqs: int, max_tokens: int, max_ctx: int, kv_pages: int = 0):
        """kv_pages: pages of 64 tokens in the attention layers' KV pool
        (0 = enough for every sequence at max_ctx)."""
        _lib.init()
        self.card = card
        self._c = card.c()
        h = C.c_void_p()
        call("ouro_stack_create", C.byref(self._c), seed, max_seqs, max_tokens, max_ctx, kv_pages, C.byref(h))
        self.handle = h.value

    @property
    def device_bytes(self) -> int:
        return int(_lib.lib().ouro_stack_device_bytes(self.handle))

    def prefill(self, tokens: DeviceBuffer, cu_seqlens: np.ndarray, next_tokens: DeviceBuffer,
                logits: DeviceBuffer | None = None, stream=None) -> None:
        cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        self._cu = cu  # the call reads it on the host
        call("ouro_stack_prefill", self.handle, tokens.ptr, cu.ctypes.data, len(cu) - 1, next_tokens.ptr,
             logits.ptr if logits is not None else None, stream)

    def decode(self, tokens: DeviceBuffer, next_tokens: DeviceBuffer, logits: DeviceBuffer | None = None,
               stream=None) -> None:
        call("ouro_stack_decode", self.handle, tokens.ptr, next_tokens.ptr,
             logits.ptr if logits is not None else None, stream)

    def free(self) -> None:
        if self.handle is not None:
            call("ouro_stack_free", self.handle)
            self.handle = None

    def __del__(self):
        try:
            if getattr(self, "handle", None) is not None and _lib._LIB is not None:
                _lib.lib().ouro_stack_free(self.handle)
                self.handle = None
        except Exception:
            pass

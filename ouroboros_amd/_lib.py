"""ctypes binding of libouro_hip.so (declared in include/ouro_hip.h).

The library is loaded from ``ouroboros_amd/lib/`` only; there is no fallback
implementation.  If it is missing, :func:`lib` raises, loudly.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libouro_hip.so"

OURO_OK = 0
STATUS_NAMES = {
    1: "OURO_ERR_INVALID_ARG",
    2: "OURO_ERR_SHAPE",
    3: "OURO_ERR_ALIGN",
    4: "OURO_ERR_KIND",
    5: "OURO_ERR_NO_DEVICE",
    6: "OURO_ERR_HIP",
    7: "OURO_ERR_NOT_INIT",
}

KIND_F32, KIND_F16, KIND_BF16, KIND_TQ1_0, KIND_TL1, KIND_I2_S, KIND_I2 = 0, 1, 30, 34, 143, 36, 0x4932
KIND_Q8_0, KIND_Q3K, KIND_Q4K, KIND_Q5K, KIND_Q6K = 8, 11, 12, 13, 14
DT_F32, DT_BF16 = 0, 1
FWHT_INVERSE = 1
GDN_L2NORM_QK, GDN_SCALE_Q, GDN_KHEAD_DIV, GDN_V_GROUPED = 1, 2, 4, 8


class OuroError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        self.code = code
        self.fn = fn
        super().__init__(f"{fn}: {STATUS_NAMES.get(code, code)}: {msg}")


vp, sz, i32, u32, f32 = C.c_void_p, C.c_size_t, C.c_int, C.c_uint, C.c_float


class StackCard(C.Structure):
    """ouro_stack_card (include/ouro_stack.h)."""
    _fields_ = [(n, C.c_int32) for n in ("n_layer", "n_embd", "n_ff", "n_vocab", "full_attention_interval",
                                          "n_head", "n_head_kv", "head_dim", "n_rot", "ssm_n_k_heads",
                                          "ssm_n_v_heads", "ssm_d_state")] + [("eps", C.c_float),
                                                                              ("rope_base", C.c_float)]

# name -> (restype, argtypes); every function of include/ouro_hip.h.
SIGNATURES = {
    "ouro_stack_create": (i32, [C.POINTER(StackCard), u32, sz, sz, sz, sz, vp]),
    "ouro_stack_free": (i32, [vp]),
    "ouro_stack_device_bytes": (sz, [vp]),
    "ouro_stack_prefill": (i32, [vp, vp, vp, sz, vp, vp, vp]),
    "ouro_stack_decode": (i32, [vp, vp, vp, vp, vp]),
    "ouro_init": (i32, [i32]),
    "ouro_shutdown": (i32, []),
    "ouro_last_error": (C.c_char_p, []),
    "ouro_abi_version": (i32, []),
    "ouro_device_count": (i32, [C.POINTER(i32)]),
    "ouro_device_arch": (i32, [C.c_char_p, sz]),
    "ouro_malloc": (i32, [C.POINTER(vp), sz]),
    "ouro_free": (i32, [vp]),
    "ouro_memcpy_htod": (i32, [vp, vp, sz]),
    "ouro_memcpy_dtoh": (i32, [vp, vp, sz]),
    "ouro_memcpy_dtod": (i32, [vp, vp, sz, vp]),
    "ouro_memset": (i32, [vp, i32, sz, vp]),
    "ouro_stream_create": (i32, [C.POINTER(vp)]),
    "ouro_stream_destroy": (i32, [vp]),
    "ouro_stream_synchronize": (i32, [vp]),
    "ouro_device_synchronize": (i32, []),
    "ouro_event_create": (i32, [C.POINTER(vp)]),
    "ouro_event_destroy": (i32, [vp]),
    "ouro_event_record": (i32, [vp, vp]),
    "ouro_event_elapsed_ms": (i32, [C.POINTER(f32), vp, vp]),
    "ouro_i2_tiled_bytes": (sz, [sz, sz]),
    "ouro_i2_tile": (i32, [vp, sz, sz, vp, vp, vp]),
    "ouro_i2s_tile": (i32, [vp, sz, sz, vp, vp]),
    "ouro_i2s_tile_mfma": (i32, [vp, sz, sz, vp, vp]),
    "ouro_act_quant_i8": (i32, [vp, i32, sz, sz, vp, vp, vp]),
    "ouro_gemm_i2": (i32, [vp, sz, sz, vp, vp, vp, sz, vp, vp, vp]),
    "ouro_gemv_i2_grouped": (i32, [vp, sz, vp, vp, sz, vp, vp, sz, sz, sz, sz, vp]),
    "ouro_i2_mfma_bytes": (sz, [sz, sz]),
    "ouro_i2_tile_mfma": (i32, [vp, sz, sz, vp, vp, vp]),
    "ouro_gemm_i2_mfma": (i32, [vp, sz, sz, vp, vp, vp, sz, vp, vp, vp]),
    "ouro_matvec_q": (i32, [vp, i32, sz, sz, vp, vp, vp]),
    "ouro_matvec_q_noalloc": (i32, [vp, i32, sz, sz, vp, vp, vp]),
    "ouro_matmul_q": (i32, [vp, i32, sz, sz, vp, sz, vp, vp]),
    "ouro_fwht_rows": (i32, [vp, i32, vp, i32, sz, sz, sz, vp, u32, vp, vp, vp]),
    "ouro_rotate_fwd": (i32, [vp, vp, sz, sz, vp]),
    "ouro_rotate_inv": (i32, [vp, vp, sz, sz, vp]),
    "ouro_delta_head_dim": (i32, [vp, sz, vp, vp, vp, f32, f32, vp, vp]),
    "ouro_gdn_decode": (i32, [vp, vp, vp, i32, vp, i32, vp, vp, vp, sz, sz, sz, sz, u32, f32, vp]),
    "ouro_gdn_chunk_workspace_bytes": (sz, [sz, sz, sz, sz, sz]),
    "ouro_gdn_layer_workspace_bytes": (sz, [sz, sz, sz, sz]),
    "ouro_gdn_layer_decode": (i32, [vp] * 11 + [sz, sz, sz, sz, u32, f32, vp, vp]),
    "ouro_gdn_chunk_prefill": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, sz, u32, f32, vp, vp]),
    "ouro_weight_upload": (i32, [i32, vp, sz, sz, sz, f32, sz, C.POINTER(vp)]),
    "ouro_weight_free": (i32, [vp]),
    "ouro_weight_payload": (vp, [vp]),
    "ouro_weight_matvec_argmax": (i32, [vp, vp, vp, vp, vp]),
    "ouro_finite_argmax": (i32, [vp, sz, vp, vp]),
    "ouro_weight_matvec": (i32, [vp, vp, vp, vp]),
    "ouro_weight_matmul": (i32, [vp, vp, sz, vp, vp]),
}

_LIB: C.CDLL | None = None


def lib() -> C.CDLL:
    """Load libouro_hip.so once and declare every entry point."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise OuroError("load", -1, f"{LIB_PATH} is missing; run __graft_entry__.build() "
                            "or `python -m ouroboros_amd.build` first")
        handle = C.CDLL(str(LIB_PATH), mode=C.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def call(name: str, *args) -> None:
    """Call a status-returning entry point; raise OuroError on failure."""
    st = getattr(lib(), name)(*args)
    if st != OURO_OK:
        msg = lib().ouro_last_error()
        raise OuroError(name, st, msg.decode() if msg else "")


_INIT_DEVICE: int | None = None


def init(device: int = -1) -> int:
    """ouro_init once per process (device -1: OURO_GPU_INDEX or 0)."""
    global _INIT_DEVICE
    if _INIT_DEVICE is None:
        call("ouro_init", device)
        _INIT_DEVICE = device
    return 0


def gpu_available() -> bool:
    """True if the HIP runtime reports at least one device (no init)."""
    if not LIB_PATH.exists():
        return False
    n = i32(0)
    return lib().ouro_device_count(C.byref(n)) == OURO_OK and n.value > 0


def env_threads() -> int:
    v = os.environ.get("OURO_N_THREADS")
    return int(v) if v and v.isdigit() and int(v) > 0 else (os.cpu_count() or 1)

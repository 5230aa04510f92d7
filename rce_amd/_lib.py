"""ctypes binding of librce_qmm.so (the C ABI of include/rce_qmm.h).

Loading fails loudly when the library has not been built: there is no CPU
fallback in this package.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "librce_qmm.so")

# Every symbol include/rce_qmm.h declares, with its ctypes signature.
P, S, U32, I, F = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_int, ctypes.c_float
STATUS = ctypes.c_int
SIGNATURES = {
    "rce_qmm_last_error": (ctypes.c_char_p, []),
    "rce_qmm_status_str": (ctypes.c_char_p, [STATUS]),
    "rce_qmm_abi_version": (U32, []),
    "rce_qmm_context_create": (STATUS, [I, P]),
    "rce_qmm_context_destroy": (None, [P]),
    "rce_qmm_context_stream": (STATUS, [P, P]),
    "rce_qmm_synchronize": (STATUS, [P]),
    "rce_qmm_supports": (I, [U32, S, I]),
    "rce_qmm_weight_from_bytes": (STATUS, [P, U32, S, S, P, S, P]),
    "rce_qmm_weight_sub_view": (STATUS, [P, S, S, S, S, P]),
    "rce_qmm_weight_destroy": (None, [P]),
    "rce_qmm_weight_info": (STATUS, [P, P, P, P, P]),
    "rce_qmm_mm_1d": (STATUS, [P, P, P, P]),
    "rce_qmm_mm_1d_serial": (STATUS, [P, P, P, P]),
    "rce_qmm_mm_batched": (STATUS, [P, P, S, P, P]),
    "rce_qmm_dequant_row": (STATUS, [P, P, S, P]),
    "rce_qmm_quantize": (STATUS, [U32, P, S, S, P, S]),
    "rce_qmm_mm_batched_dev": (STATUS, [P, P, U32, S, P, P, I, P]),
    "rce_qmm_mm_batched_dev_noalloc": (STATUS, [P, P, U32, S, P, P, I, P]),
    "rce_qmm_moe_router": (STATUS, [P, S, S, S, I, P, P]),
    "rce_qmm_moe_ffn_dev": (STATUS, [P, P, P, S, P, S, P, P, S, P, I, P]),
    "rce_qmm_moe_swiglu_dev": (STATUS, [P, P, P, P, S, P, S, P, P, S, P, I, P]),
    "rce_qmm_llama_create": (STATUS, [P, P, P, P, P, P, I, P]),
    "rce_qmm_llama_destroy": (None, [P]),
    "rce_qmm_llama_reset": (STATUS, [P]),
    "rce_qmm_llama_pos": (STATUS, [P, P]),
    "rce_qmm_llama_forward_token": (STATUS, [P, ctypes.c_int32, P]),
    "rce_qmm_llama_forward_embedding": (STATUS, [P, P, P]),
    "rce_qmm_llama_forward_token_dev": (STATUS, [P, P, P, P]),
    "rce_qmm_llama_check": (STATUS, [P]),
    "rce_qmm_gguf_parse": (STATUS, [P, S, P]),
    "rce_qmm_gguf_open": (STATUS, [ctypes.c_char_p, P]),
    "rce_qmm_gguf_close": (None, [P]),
    "rce_qmm_gguf_header": (STATUS, [P, P, P, P, P, P]),
    "rce_qmm_gguf_metadata": (STATUS, [P, S, P, P, P, P]),
    "rce_qmm_gguf_find_metadata": (STATUS, [P, ctypes.c_char_p, P]),
    "rce_qmm_gguf_tensor": (STATUS, [P, S, P, P, P, P, P, P]),
    "rce_qmm_gguf_find_tensor": (STATUS, [P, ctypes.c_char_p, P]),
    "rce_qmm_weight_from_gguf": (STATUS, [P, P, ctypes.c_char_p, S, S, P]),
    "rce_qmm_gguf_read_f32": (STATUS, [P, ctypes.c_char_p, P, S]),
    "rce_qmm_dtype_for_qmm_id": (U32, [S]),
    "rce_qmm_hip_cost_prior": (None, [P, P, P]),
    "rce_qmm_hip_cost": (STATUS, [P, S, P, S, ctypes.c_double, ctypes.c_double, ctypes.c_double, P]),
    "rce_qmm_energy_read": (STATUS, [I, P, P]),
    "rce_qmm_read_ceiling_dev": (STATUS, [P, P, S, P, I, P]),
    "rce_qmm_dev_alloc": (STATUS, [P, S, P]),
    "rce_qmm_dev_free": (STATUS, [P, P]),
    "rce_qmm_memcpy_h2d": (STATUS, [P, P, P, S]),
    "rce_qmm_memcpy_d2h": (STATUS, [P, P, P, S]),
}

_lib = None


class QmmError(RuntimeError):
    """A non-OK rce_qmm_status, with the library's last-error text."""

    def __init__(self, status: int, msg: str):
        super().__init__(f"rce_qmm status {status}: {msg}")
        self.status = status


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m rce_amd.build` "
                "(or __graft_entry__.build()); there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != 0:
        raise QmmError(status, lib().rce_qmm_last_error().decode(errors="replace"))

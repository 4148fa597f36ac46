"""ctypes binding of libcq35.so (the C ABI declared in include/cq35.h)."""
from __future__ import annotations

import ctypes
import os

from .config import CConfig

# CQ35_LIBRARY selects another in-tree build (the phase-trace library)
LIBRARY = os.environ.get("CQ35_LIBRARY") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libcq35.so")
_lib = None


class CQ35Error(RuntimeError):
    """A failed cq35 call: `code` is the negative CQ35_E* value."""

    def __init__(self, code: int, message: str):
        super().__init__(f"cq35 error {code}: {message}")
        self.code = code


class TensorInfo(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
                ("bytes", ctypes.c_int64)]


def load():
    """Load the in-tree library; raise loudly when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIBRARY):
        raise RuntimeError(
            f"{LIBRARY} is missing: build it with `python -m cq35._build` or "
            "`python -c 'import __graft_entry__; __graft_entry__.build()'`")
    l = ctypes.CDLL(LIBRARY)
    P, I64, I32, U64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_uint64
    PC = ctypes.POINTER(CConfig)
    sig = {
        "cq35_last_error": ([], ctypes.c_char_p),
        "cq35_abi_version": ([], ctypes.c_int),
        "cq35_config_validate": ([PC], ctypes.c_int),
        "cq35_weight_count": ([PC, ctypes.POINTER(I64)], ctypes.c_int),
        "cq35_weight_info": ([PC, I64, ctypes.POINTER(TensorInfo)], ctypes.c_int),
        "cq35_model_create": ([PC, ctypes.POINTER(P), ctypes.c_int, ctypes.POINTER(P)], ctypes.c_int),
        "cq35_model_create_synthetic": ([PC, U64, ctypes.POINTER(P)], ctypes.c_int),
        "cq35_model_free": ([P], ctypes.c_int),
        "cq35_model_config": ([P, PC], ctypes.c_int),
        "cq35_model_weight_bytes": ([P, ctypes.POINTER(I64)], ctypes.c_int),
        "cq35_model_read_weight": ([P, I64, P, I64], ctypes.c_int),
        "cq35_session_init": ([P, I64, ctypes.POINTER(P)], ctypes.c_int),
        "cq35_session_free": ([P], ctypes.c_int),
        "cq35_step": ([P, P, I64, I64, I64, ctypes.POINTER(U64), P], ctypes.c_int),
        "cq35_session_copy": ([P, ctypes.POINTER(P)], ctypes.c_int),
        "cq35_session_state_bytes": ([P, ctypes.c_int, ctypes.POINTER(I64)], ctypes.c_int),
        "cq35_session_export_state": ([P, ctypes.c_int, P, I64], ctypes.c_int),
        "cq35_session_import_state": ([P, ctypes.c_int, P, I64], ctypes.c_int),
        "cq35_session_time_kernel": ([P, ctypes.c_int], ctypes.c_int),
        "cq35_session_kernel_time": ([P, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(I64)], ctypes.c_int),
        "cq35_kernel_class_name": ([ctypes.c_int], ctypes.c_char_p),
        "cq35_kernel_class_count": ([], ctypes.c_int),
        "cq35_session_set_graph": ([P, ctypes.c_int], ctypes.c_int),
        "cq35_session_set_persistent": ([P, ctypes.c_int], ctypes.c_int),
        "cq35_session_persistent": ([P, ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
        "cq35_session_set_matrix_prefill": ([P, ctypes.c_int], ctypes.c_int),
        "cq35_session_matrix_prefill": ([P, ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
        "cq35_session_set_matrix_decode": ([P, ctypes.c_int], ctypes.c_int),
        "cq35_session_matrix_decode": ([P, ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
        "cq35_numeric_exp": ([ctypes.c_float], ctypes.c_float),
        "cq35_numeric_sqrt": ([ctypes.c_float], ctypes.c_float),
        "cq35_numeric_softplus": ([ctypes.c_float], ctypes.c_float),
        "cq35_numeric_sincos": ([ctypes.c_float, ctypes.POINTER(ctypes.c_float),
                                 ctypes.POINTER(ctypes.c_float)], None),
        "cq35_device_numeric": ([ctypes.c_int, P, P, I64], ctypes.c_int),
        "cq35_device_gemv": ([P, P, I64, I64, ctypes.c_int, P], ctypes.c_int),
        "cq35_device_matrix_gemm": ([P, P, P, P, I64, I64, I64, ctypes.c_int, ctypes.c_int, P],
                                    ctypes.c_int),
        "cq35_device_matrix_attention": ([P, P, P, P, I64, I64, ctypes.c_int, ctypes.c_int, ctypes.c_int, P],
                                         ctypes.c_int),
        "cq35_step_batch": ([ctypes.POINTER(P), P, P, I64, P, P], ctypes.c_int),
        "cq35_gguf_config": ([ctypes.c_char_p, PC], ctypes.c_int),
        "cq35_gguf_validate": ([ctypes.c_char_p, PC], ctypes.c_int),
        "cq35_model_load_gguf": ([ctypes.c_char_p, ctypes.POINTER(P)], ctypes.c_int),
        "cq35_gguf_tensor_name": ([PC, I64, ctypes.c_char_p, I64], ctypes.c_int),
        "cq35_step_static": ([P, P, I64, U64, I64, P, ctypes.POINTER(U64), P], ctypes.c_int),
        "cq35_session_set_attention_split": ([P, I64], ctypes.c_int),
        "cq35_session_attention_split": ([P, ctypes.POINTER(I64)], ctypes.c_int),
        "cq35_session_phase_trace": ([P, P, I64, ctypes.POINTER(I64), ctypes.POINTER(I64)], ctypes.c_int),
    }
    for name, (args, res) in sig.items():
        f = getattr(l, name)
        f.argtypes = args
        f.restype = res
    _lib = l
    return l


def check(rc: int) -> None:
    if rc != 0:
        raise CQ35Error(rc, load().cq35_last_error().decode(errors="replace"))


EXPORTED = [
    "cq35_last_error", "cq35_abi_version", "cq35_config_validate", "cq35_weight_count",
    "cq35_weight_info", "cq35_model_create", "cq35_model_create_synthetic", "cq35_model_free",
    "cq35_model_config", "cq35_model_weight_bytes", "cq35_model_read_weight", "cq35_session_init",
    "cq35_session_free", "cq35_step", "cq35_session_copy", "cq35_session_state_bytes",
    "cq35_session_export_state", "cq35_session_import_state", "cq35_session_time_kernel",
    "cq35_session_kernel_time", "cq35_kernel_class_name", "cq35_kernel_class_count",
    "cq35_session_set_graph", "cq35_session_set_persistent", "cq35_session_persistent",
    "cq35_session_set_matrix_prefill", "cq35_session_matrix_prefill",
    "cq35_session_set_matrix_decode", "cq35_session_matrix_decode",
    "cq35_numeric_exp", "cq35_numeric_sqrt", "cq35_numeric_softplus",
    "cq35_numeric_sincos", "cq35_device_numeric", "cq35_device_gemv", "cq35_device_matrix_gemm",
    "cq35_device_matrix_attention",
    "cq35_gguf_config", "cq35_gguf_validate", "cq35_model_load_gguf", "cq35_gguf_tensor_name",
    "cq35_step_batch", "cq35_step_static", "cq35_session_set_attention_split",
    "cq35_session_attention_split", "cq35_session_phase_trace",
]

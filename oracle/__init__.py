"""ctypes front end of the CPU restatement in ``oracle/oracle.c``.

Test infrastructure only: the parity checker and the CPU baseline. Nothing in
the shipped library imports this module; only ``tests/``, ``bench.py``'s
``cpu_baseline`` leg and ``__graft_entry__.smoke()`` may use it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

FIELDS = [
    ("moe", ctypes.c_int32), ("vocab", ctypes.c_int32), ("hidden", ctypes.c_int32),
    ("intermediate", ctypes.c_int32), ("layers", ctypes.c_int32), ("q_heads", ctypes.c_int32),
    ("kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("rope_dim", ctypes.c_int32),
    ("eps", ctypes.c_float), ("theta", ctypes.c_float), ("experts", ctypes.c_int32),
    ("top_k", ctypes.c_int32), ("shared_intermediate", ctypes.c_int32),
    ("full_interval", ctypes.c_int32), ("key_heads", ctypes.c_int32),
    ("key_dim", ctypes.c_int32), ("value_heads", ctypes.c_int32),
    ("value_dim", ctypes.c_int32), ("tied", ctypes.c_int32),
]


class OxConfig(ctypes.Structure):
    _fields_ = FIELDS


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "liboracle.so"],
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        l = ctypes.CDLL(_LIB_PATH)
        P, I64, I32, U64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_uint64
        l.ox_weight_count.argtypes = [ctypes.POINTER(OxConfig)]
        l.ox_weight_count.restype = I64
        l.ox_weight_info.argtypes = [ctypes.POINTER(OxConfig), I64, ctypes.POINTER(I32),
                                     ctypes.POINTER(I64), ctypes.POINTER(I64), ctypes.POINTER(I32)]
        l.ox_weight_info.restype = ctypes.c_int
        for name in ["ox_exp", "ox_silu", "ox_sigmoid", "ox_softplus", "ox_sqrt"]:
            getattr(l, name).argtypes = [ctypes.c_float]
            getattr(l, name).restype = ctypes.c_float
        l.ox_sincos.argtypes = [ctypes.c_float, ctypes.POINTER(ctypes.c_float),
                                ctypes.POINTER(ctypes.c_float)]
        l.ox_f2bf.argtypes = [ctypes.c_float]
        l.ox_f2bf.restype = ctypes.c_uint16
        l.ox_dot_width.argtypes = [P, P, I64, ctypes.c_int]
        l.ox_dot_width.restype = ctypes.c_float
        l.ox_dot_width_f32w.argtypes = [P, P, I64, ctypes.c_int]
        l.ox_dot_width_f32w.restype = ctypes.c_float
        l.ox_dot_b256.argtypes = [P, P, I64]
        l.ox_dot_b256.restype = ctypes.c_float
        l.ox_fill_tensor.argtypes = [ctypes.POINTER(OxConfig), U64, I64, P]
        l.ox_mix64.argtypes = [U64]
        l.ox_mix64.restype = U64
        l.ox_model_create.argtypes = [ctypes.POINTER(OxConfig), ctypes.POINTER(P)]
        l.ox_model_create.restype = P
        l.ox_model_free.argtypes = [P]
        l.ox_session_create.argtypes = [P, I64]
        l.ox_session_create.restype = P
        l.ox_session_free.argtypes = [P]
        l.ox_cache_elements.argtypes = [ctypes.POINTER(OxConfig), I64]
        l.ox_cache_elements.restype = I64
        l.ox_session_cache.argtypes = [P]
        l.ox_session_cache.restype = ctypes.POINTER(ctypes.c_uint16)
        l.ox_session_shadow.argtypes = [P]
        l.ox_session_shadow.restype = ctypes.POINTER(ctypes.c_float)
        l.ox_session_last_ids.argtypes = [P]
        l.ox_session_last_ids.restype = ctypes.POINTER(ctypes.c_int64)
        l.ox_step.argtypes = [P, P, I64, I64, ctypes.POINTER(U64), P]
        l.ox_step.restype = ctypes.c_int
        l.ox_set_threads.argtypes = [ctypes.c_int]
        l.ox_set_plant.argtypes = [ctypes.c_int]
        l.ox_k_normalize.argtypes = [P, P, I64, I64, ctypes.c_float, P]
        l.ox_k_prepare_heads.argtypes = [P, I64, P, P, I64, P]
        l.ox_k_rope.argtypes = [P, I64, P, I64, P]
        l.ox_k_conv.argtypes = [P, P, I64, P, P, P]
        l.ox_k_l2.argtypes = [P, ctypes.c_int, ctypes.c_int, P]
        l.ox_k_delta.argtypes = [P, P, P, P, P, P, P, P, P, P, P]
        l.ox_k_gated_norm.argtypes = [P, P, P, P, P]
        l.ox_k_attention.argtypes = [P, ctypes.c_int, P, P, I64, P, I64, P]
        l.ox_session_set_split_keys.argtypes = [P, I64]
        l.ox_k_select.argtypes = [P, I64, I64, P, P]
        l.ox_k_argmax.argtypes = [P, I64]
        l.ox_k_argmax.restype = U64
        l.ox_moe_route.argtypes = [P, P, P, I64, I64, I64, P, P, P]
        _lib = l
    return _lib


# Planted mistakes (oracle.h OX_PLANT_*): switched on only by the pinning
# tests, to show that a comparison fails for that mistake.
PLANTS = {
    "rope_pairing": 1, "rope_sign": 2, "rope_freq_hd": 3, "qk_norm_swap": 4,
    "conv_tap_order": 5, "delta_scale": 6, "l2_whole": 7, "gated_sum": 8,
    "attn_scale": 9, "gqa_map": 10, "norm_weight": 11, "key_head": 12,
    "delta_pred_decay": 13, "select_tie_high": 14, "select_ascending": 15,
    "prob_unnormalised": 16, "softmax_all": 17, "shared_gate": 18, "argmax_last": 19,
}


class planted:
    """Context manager: the restatement runs with one planted mistake."""

    def __init__(self, name):
        self.code = PLANTS[name] if name else 0

    def __enter__(self):
        lib().ox_set_plant(self.code)
        return self

    def __exit__(self, *exc):
        lib().ox_set_plant(0)
        return False


def make_config(cfg: dict) -> OxConfig:
    c = OxConfig()
    for name, _ in FIELDS:
        setattr(c, name, cfg[name])
    return c


# ------------------------------------------------------------ scalar helpers

def exp(x: float) -> float:
    return lib().ox_exp(x)


def bf16_round(values: np.ndarray) -> np.ndarray:
    """F32 -> BF16 bits, round-to-nearest-even, NaNs quieted (src/weights.rs:213-221)."""
    f = np.ascontiguousarray(values, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    rounded[nan] = ((u[nan] >> 16).astype(np.uint16) | 0x0040)
    return rounded


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def dot_width(x: np.ndarray, w: np.ndarray, width: int) -> float:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    if w.dtype == np.float32:
        w = np.ascontiguousarray(w)
        return lib().ox_dot_width_f32w(x.ctypes.data, w.ctypes.data, len(x) // 2, width)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    return lib().ox_dot_width(x.ctypes.data, w.ctypes.data, len(x) // 2, width)


def dot_b256(x: np.ndarray, w: np.ndarray) -> float:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    return lib().ox_dot_b256(x.ctypes.data, w.ctypes.data, len(x) // 2)


def select(logits: np.ndarray, k: int):
    """Top-k ids (rank order) and routing weights over F32 router logits."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    ids = np.zeros(k, dtype=np.int64)
    probs = np.zeros(k, dtype=np.float32)
    lib().ox_k_select(lg.ctypes.data, lg.size, k, ids.ctypes.data, probs.ctypes.data)
    return ids, probs


def argmax(logits: np.ndarray) -> int:
    """Greedy token over BF16 logit bits."""
    lg = np.ascontiguousarray(logits, dtype=np.uint16)
    return int(lib().ox_k_argmax(lg.ctypes.data, lg.size))


# ------------------------------------------------------------- weights/model

def weight_specs(cfg: dict):
    c = make_config(cfg)
    l = lib()
    out = []
    for i in range(l.ox_weight_count(ctypes.byref(c))):
        d, k = ctypes.c_int32(), ctypes.c_int32()
        r, co = ctypes.c_int64(), ctypes.c_int64()
        rc = l.ox_weight_info(ctypes.byref(c), i, ctypes.byref(d), ctypes.byref(r),
                              ctypes.byref(co), ctypes.byref(k))
        assert rc == 0
        out.append(("bf16" if d.value == 0 else "f32", r.value, co.value, k.value))
    return out


def synthetic_weights(cfg: dict, seed: int):
    """Materialise every tensor of the weight ABI with the synthetic generator."""
    c = make_config(cfg)
    arrays = []
    specs = weight_specs(cfg)
    for i, (dtype, rows, cols, _kind) in enumerate(specs):
        if cfg["tied"] and i == len(specs) - 1:
            arrays.append(arrays[0])
            continue
        a = np.empty(rows * cols, dtype=np.uint16 if dtype == "bf16" else np.float32)
        lib().ox_fill_tensor(ctypes.byref(c), seed, i, a.ctypes.data)
        arrays.append(a)
    return arrays


class Model:
    def __init__(self, cfg: dict, weights):
        self.cfg = dict(cfg)
        self._c = make_config(cfg)
        self.weights = weights
        ptrs = (ctypes.c_void_p * len(weights))(*[w.ctypes.data for w in weights])
        self._ptrs = ptrs
        self._h = lib().ox_model_create(ctypes.byref(self._c), ptrs)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().ox_model_free(self._h)
            self._h = None

    def session(self, capacity: int) -> "Session":
        return Session(self, capacity)


class Session:
    def __init__(self, model: Model, capacity: int):
        self.model = model
        self.capacity = capacity
        self._h = lib().ox_session_create(model._h, capacity)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().ox_session_free(self._h)
            self._h = None

    def step(self, tokens, start: int, want_logits: bool = True):
        toks = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint64))
        nxt = ctypes.c_uint64()
        logits = np.empty(self.model.cfg["vocab"], dtype=np.uint16) if want_logits else None
        rc = lib().ox_step(self._h, toks.ctypes.data, len(toks), start, ctypes.byref(nxt),
                           logits.ctypes.data if want_logits else None)
        if rc != 0:
            raise RuntimeError(f"oracle step failed with code {rc}")
        return int(nxt.value), logits

    def cache(self) -> np.ndarray:
        n = lib().ox_cache_elements(ctypes.byref(self.model._c), self.capacity)
        return np.ctypeslib.as_array(lib().ox_session_cache(self._h), shape=(n,)).copy()

    def import_cache(self, data: np.ndarray) -> None:
        """Overwrite the BF16 session state (same layout as ``cache()``)."""
        n = lib().ox_cache_elements(ctypes.byref(self.model._c), self.capacity)
        src = np.ascontiguousarray(data, dtype=np.uint16).reshape(-1)
        if src.size != n:
            raise ValueError(f"state has {src.size} elements, expected {n}")
        np.ctypeslib.as_array(lib().ox_session_cache(self._h), shape=(n,))[:] = src

    def set_split_keys(self, keys: int) -> None:
        """Decode attention over more than `keys` keys as four merged splits
        (0: the reference's single chain at every length)."""
        lib().ox_session_set_split_keys(self._h, keys)

    def last_ids(self) -> np.ndarray:
        c = self.model.cfg
        n = c["layers"] * max(c["top_k"], 1)
        return np.ctypeslib.as_array(lib().ox_session_last_ids(self._h), shape=(n,)).copy()

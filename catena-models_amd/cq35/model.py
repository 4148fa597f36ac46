"""Host-side mirror of catena-models' Model / Session API (src/model.rs) over
the cq35 C ABI. Method names, argument meaning and error behaviour follow the
reference:

  Model.session(capacity)                 src/model.rs:192-206
  Session.prefill_next_token(tokens)      src/model.rs:484-492
  Session.decode_next_token(token)        src/model.rs:494-502
  Session.append_next_token(tokens)       src/model.rs:449-456
  Session.{prefill,decode,append}_logits  src/model.rs:458-482
  Session.into_checkpoint()               src/model.rs:431-446
  Model.resume_checkpoint(checkpoint)     src/model.rs:209-246
  Model.logits / Model.next_token         src/model.rs:187-190

A failed step leaves the session unusable, like the reference's `state.take()`
(src/model.rs:711-730).
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import numpy as np

from . import _lib
from ._lib import CQ35Error, check
from .config import CConfig, from_c, preset, to_c


class Model:
    def __init__(self, handle: int, cfg: dict):
        self._h = ctypes.c_void_p(handle)
        self.cfg = dict(cfg)

    # -- construction ---------------------------------------------------
    @classmethod
    def synthetic(cls, cfg, seed: int = 0) -> "Model":
        """Weights generated on the device by the library's seeded generator."""
        cfg = preset(cfg) if isinstance(cfg, str) else dict(cfg)
        lib = _lib.load()
        out = ctypes.c_void_p()
        c = to_c(cfg)
        check(lib.cq35_model_create_synthetic(ctypes.byref(c), seed, ctypes.byref(out)))
        return cls(out.value, cfg)

    @classmethod
    def load_gguf(cls, path: str) -> "Model":
        """A GGUF checkpoint (one file, any shard of a set, or a directory):
        configuration from its metadata, tensors checked against weight_specs
        and copied into HBM (Model::load_gguf, src/model.rs:43, 81-153)."""
        lib = _lib.load()
        out = ctypes.c_void_p()
        check(lib.cq35_model_load_gguf(str(path).encode(), ctypes.byref(out)))
        m = cls(out.value, {})
        m.cfg = m.config()
        return m

    @classmethod
    def from_arrays(cls, cfg: dict, arrays: Sequence[np.ndarray]) -> "Model":
        """Upload host tensors given in weight_specs order (src/spec.rs:443-712)."""
        lib = _lib.load()
        c = to_c(cfg)
        ptrs = (ctypes.c_void_p * len(arrays))(*[a.ctypes.data for a in arrays])
        out = ctypes.c_void_p()
        check(lib.cq35_model_create(ctypes.byref(c), ptrs, 0, ctypes.byref(out)))
        m = cls(out.value, cfg)
        m._keep = arrays
        return m

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            _lib.load().cq35_model_free(self._h)
            self._h = ctypes.c_void_p()

    def config(self) -> dict:
        c = CConfig()
        check(_lib.load().cq35_model_config(self._h, ctypes.byref(c)))
        return from_c(c)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- queries ----------------------------------------------------------
    @property
    def vocabulary_size(self) -> int:
        return self.cfg["vocab"]

    def weight_bytes(self) -> int:
        b = ctypes.c_int64()
        check(_lib.load().cq35_model_weight_bytes(self._h, ctypes.byref(b)))
        return b.value

    def read_weight(self, index: int) -> np.ndarray:
        info = weight_info(self.cfg, index)
        dtype = np.uint16 if info.dtype == 0 else np.float32
        a = np.empty(info.rows * info.cols, dtype=dtype)
        check(_lib.load().cq35_model_read_weight(self._h, index, a.ctypes.data, info.bytes))
        return a

    # -- sessions ---------------------------------------------------------
    def session(self, capacity: int) -> "Session":
        if capacity <= 0:
            raise ValueError("cache capacity must be non-zero")
        out = ctypes.c_void_p()
        check(_lib.load().cq35_session_init(self._h, capacity, ctypes.byref(out)))
        return Session(self, out.value, capacity, 0)

    def resume_checkpoint(self, checkpoint: "SessionCheckpoint") -> "Session":
        if checkpoint.model is not self:
            raise ValueError("session checkpoint belongs to another loaded model")
        out = ctypes.c_void_p()
        check(_lib.load().cq35_session_copy(checkpoint._h, ctypes.byref(out)))
        return Session(self, out.value, checkpoint.capacity, checkpoint.position)

    def logits(self, tokens: Sequence[int]) -> np.ndarray:
        return self.session(len(tokens)).prefill_logits(tokens)

    def next_token(self, tokens: Sequence[int]) -> int:
        return self.session(len(tokens)).prefill_next_token(tokens)


def weight_info(cfg: dict, index: int):
    info = _lib.TensorInfo()
    c = to_c(cfg)
    check(_lib.load().cq35_weight_info(ctypes.byref(c), index, ctypes.byref(info)))
    return info


def decode_batch(sessions: Sequence["Session"], tokens: Sequence[int], logits: bool = False):
    """One decode step for each session (cq35_step_batch): the same next
    tokens as stepping them one by one (sessions of one model and capacity
    share each layer's weight pass; with matrix-core decode selected on every
    session the products run on MFMA). With logits=True,
    also returns the BF16 logits as a [sessions, vocab] uint16 array."""
    n = len(sessions)
    if n == 0:
        return []
    if len(tokens) != n:
        raise ValueError("one token per session")
    for s in sessions:
        if not s._alive:
            raise RuntimeError("session state unavailable after failed execution")
        if s.position <= 0:
            raise ValueError("decode requires a completed prefill")
        if s.position + 1 > s.capacity:
            raise ValueError("token range exceeds cache capacity")
    handles = (ctypes.c_void_p * n)(*[s._h.value for s in sessions])
    toks = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint64))
    starts = np.ascontiguousarray(np.asarray([s.position for s in sessions], dtype=np.int64))
    out = np.zeros(n, dtype=np.uint64)
    lg = np.empty((n, sessions[0].model.cfg["vocab"]), dtype=np.uint16) if logits else None
    rc = _lib.load().cq35_step_batch(handles, toks.ctypes.data, starts.ctypes.data, n, out.ctypes.data,
                                     lg.ctypes.data if logits else None)
    if rc != 0:
        if rc in (-3, -5):  # a step may have failed part-way: no session of the batch is trusted
            for s in sessions:
                s._alive = False
        check(rc)
    for s in sessions:
        s.position += 1
    toks_out = [int(x) for x in out]
    return (toks_out, lg) if logits else toks_out


def gguf_config(path: str) -> dict:
    """Model configuration from GGUF metadata (read_gguf_model_config,
    src/checkpoint.rs:376-404); no GPU needed."""
    c = CConfig()
    check(_lib.load().cq35_gguf_config(str(path).encode(), ctypes.byref(c)))
    return from_c(c)


def gguf_validate(path: str, cfg: dict | None = None) -> None:
    """validate_gguf_tensors (src/checkpoint.rs:406-414): raises CQ35Error
    when the inventory, a shape, a dtype or a byte range is wrong."""
    c = to_c(cfg) if cfg is not None else None
    check(_lib.load().cq35_gguf_validate(str(path).encode(), ctypes.byref(c) if c is not None else None))


def gguf_tensor_name(cfg: dict, index: int) -> str:
    buf = ctypes.create_string_buffer(256)
    c = to_c(cfg)
    check(_lib.load().cq35_gguf_tensor_name(ctypes.byref(c), index, buf, 256))
    return buf.value.decode()


def weight_count(cfg: dict) -> int:
    n = ctypes.c_int64()
    c = to_c(cfg)
    check(_lib.load().cq35_weight_count(ctypes.byref(c), ctypes.byref(n)))
    return n.value


class Session:
    def __init__(self, model: Model, handle: int, capacity: int, position: int):
        self.model = model
        self._h = ctypes.c_void_p(handle)
        self.capacity = capacity
        self.position = position
        self._alive = True

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            _lib.load().cq35_session_free(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- the forward call (src/model.rs:692-731) --------------------------
    def _forward(self, tokens: Sequence[int], want_logits: bool):
        if not self._alive:
            raise RuntimeError("session state unavailable after failed execution")
        toks = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint64).reshape(-1))
        if len(toks) == 0 or self.position + len(toks) > self.capacity:
            raise ValueError("token range exceeds cache capacity")
        if np.any(toks >= self.model.vocabulary_size):
            raise ValueError("token ID outside vocabulary")
        nxt = ctypes.c_uint64()
        logits = np.empty(self.model.vocabulary_size, dtype=np.uint16) if want_logits else None
        rc = _lib.load().cq35_step(self._h, toks.ctypes.data, len(toks), self.position,
                                   self.capacity, ctypes.byref(nxt),
                                   logits.ctypes.data if want_logits else None)
        if rc != 0:
            if rc in (-3, -5):
                self._alive = False
            check(rc)
        self.position += len(toks)
        return logits, int(nxt.value)

    def append_next_token(self, tokens: Sequence[int]) -> int:
        return self._forward(tokens, False)[1]

    def append_logits(self, tokens: Sequence[int]) -> np.ndarray:
        return read_logits(self._forward(tokens, True)[0])

    def prefill_logits(self, tokens: Sequence[int]) -> np.ndarray:
        if self.position != 0:
            raise ValueError("a session can only be prefilled once")
        return read_logits(self._forward(tokens, True)[0])

    def decode_logits(self, token: int) -> np.ndarray:
        if self.position <= 0:
            raise ValueError("decode requires a completed prefill")
        return read_logits(self._forward([token], True)[0])

    def prefill_next_token(self, tokens: Sequence[int]) -> int:
        if self.position != 0:
            raise ValueError("a session can only be prefilled once")
        return self._forward(tokens, False)[1]

    def decode_next_token(self, token: int) -> int:
        if self.position <= 0:
            raise ValueError("decode requires a completed prefill")
        return self._forward([token], False)[1]

    def step_raw(self, tokens: Sequence[int], want_logits: bool = True):
        """(BF16 logits bits, next token) of one call, without the checks."""
        return self._forward(tokens, want_logits)

    # -- state ------------------------------------------------------------
    def state_bytes(self, which: int) -> int:
        b = ctypes.c_int64()
        check(_lib.load().cq35_session_state_bytes(self._h, which, ctypes.byref(b)))
        return b.value

    def export_state(self, which: int = 0) -> np.ndarray:
        """which 0: BF16 cache bits; 1: F32 DeltaNet shadow; 2 (MoE): int32
        [layers, top_k] expert ids chosen for the last call's final token."""
        n = self.state_bytes(which)
        dtype = {0: np.uint16, 1: np.float32, 2: np.int32}[which]
        a = np.empty(n // np.dtype(dtype).itemsize, dtype=dtype)
        check(_lib.load().cq35_session_export_state(self._h, which, a.ctypes.data, n))
        if which == 2:
            a = a.reshape(self.model.cfg["layers"], -1)
        return a

    def router_ids(self) -> np.ndarray:
        """Per-layer top-k expert ids (rank order) of the last call's final token."""
        return self.export_state(2)

    def import_state(self, which: int, data: np.ndarray) -> None:
        a = np.ascontiguousarray(data)
        check(_lib.load().cq35_session_import_state(self._h, which, a.ctypes.data, a.nbytes))

    def into_checkpoint(self) -> "SessionCheckpoint":
        if not self._alive:
            raise RuntimeError("session state is unavailable after an inference error")
        cp = SessionCheckpoint(self.model, self._h, self.capacity, self.position)
        self._h = ctypes.c_void_p()
        self._alive = False
        return cp

    def set_graph(self, enabled: bool) -> None:
        check(_lib.load().cq35_session_set_graph(self._h, 1 if enabled else 0))

    def set_persistent(self, enabled: bool) -> None:
        """Decode steps through the persistent one-launch kernel (MoE shapes
        it covers; the default there) or the per-kernel launch sequence."""
        check(_lib.load().cq35_session_set_persistent(self._h, 1 if enabled else 0))

    MATRIX_PROJECTIONS = 1
    MATRIX_EXPERTS = 2
    MATRIX_ATTENTION = 4

    def set_attention_split(self, keys: int) -> None:
        """Decode attention over more than `keys` cached keys as at most 128
        ranges of equal tile counts, each an online recurrence of its own,
        merged in ascending order (0: the reference's single chain at every
        length)."""
        check(_lib.load().cq35_session_set_attention_split(self._h, keys))

    @property
    def attention_split(self) -> int:
        k = ctypes.c_int64()
        check(_lib.load().cq35_session_attention_split(self._h, ctypes.byref(k)))
        return k.value

    def set_matrix_prefill(self, components: int) -> None:
        """Run these components of multi-token calls on MFMA (hardware
        accumulation order; 0 = the exact SIMT path): MATRIX_PROJECTIONS,
        MATRIX_EXPERTS, MATRIX_ATTENTION or any combination (the reference's
        wmma_prefill scopes)."""
        check(_lib.load().cq35_session_set_matrix_prefill(self._h, int(components)))

    @property
    def matrix_prefill(self) -> int:
        v = ctypes.c_int()
        check(_lib.load().cq35_session_matrix_prefill(self._h, ctypes.byref(v)))
        return v.value

    def set_matrix_decode(self, enabled: bool) -> None:
        """Let cq35_step_batch run the weight-shared step's products on MFMA
        (tolerance-level) when every session of the batch has this set; a
        batch with any session unset takes the exact products."""
        check(_lib.load().cq35_session_set_matrix_decode(self._h, 1 if enabled else 0))

    @property
    def matrix_decode(self) -> bool:
        v = ctypes.c_int()
        check(_lib.load().cq35_session_matrix_decode(self._h, ctypes.byref(v)))
        return bool(v.value)

    @property
    def persistent(self) -> bool:
        v = ctypes.c_int()
        check(_lib.load().cq35_session_persistent(self._h, ctypes.byref(v)))
        return bool(v.value)

    def time_kernel(self, kernel_class: int) -> None:
        check(_lib.load().cq35_session_time_kernel(self._h, kernel_class))

    def kernel_time(self):
        ms, n = ctypes.c_double(), ctypes.c_int64()
        check(_lib.load().cq35_session_kernel_time(self._h, ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value


class SessionCheckpoint:
    """Immutable frozen state; resumable only by its own model."""

    def __init__(self, model: Model, handle, capacity: int, position: int):
        self.model = model
        self._h = handle
        self.capacity = capacity
        self.position = position

    def byte_len(self) -> int:
        """Device bytes the frozen state holds (cache + F32 workspace)."""
        total = 0
        for which in (0, 1):
            b = ctypes.c_int64()
            check(_lib.load().cq35_session_state_bytes(self._h, which, ctypes.byref(b)))
            total += b.value
        return total

    def __del__(self):
        try:
            if self._h and self._h.value:
                _lib.load().cq35_session_free(self._h)
        except Exception:
            pass


def read_logits(bits: np.ndarray) -> np.ndarray:
    """BF16 bits -> F32 logits; non-finite logits are an error (src/model.rs:734-750)."""
    f = (bits.astype(np.uint32) << 16).view(np.float32)
    if not np.all(np.isfinite(f)):
        raise ValueError("qwen3 returned non-finite logits")
    return f


def kernel_classes() -> list[str]:
    lib = _lib.load()
    return [lib.cq35_kernel_class_name(i).decode() for i in range(lib.cq35_kernel_class_count())]

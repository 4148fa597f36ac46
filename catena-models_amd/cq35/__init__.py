"""cq35: MI355X-native Qwen3.5/3.6 token loop (hand-written gfx950 HIP
kernels behind a C ABI) with a host API mirroring catena-models' Model /
Session (src/model.rs)."""
from .config import PRESETS, bytes_per_token, derived, is_full, preset
from .model import (Model, Session, SessionCheckpoint, decode_batch, gguf_config, gguf_tensor_name, gguf_validate,
                    kernel_classes, read_logits, weight_count, weight_info)
from ._lib import CQ35Error, LIBRARY, load

# decode attention over more cached keys than this runs split-K by default
# (include/cq35.h CQ35_SPLIT_KEYS_DEFAULT)
SPLIT_KEYS_DEFAULT = 8192

__all__ = [
    "PRESETS", "bytes_per_token", "derived", "is_full", "preset", "Model", "Session",
    "SessionCheckpoint", "decode_batch", "gguf_config", "gguf_tensor_name", "gguf_validate", "kernel_classes",
    "read_logits", "weight_count", "weight_info",
    "CQ35Error", "LIBRARY", "load", "SPLIT_KEYS_DEFAULT",
]

"""Model configurations of the token loop (the subset of ModelConfig the decode
step reads, src/spec.rs:33-62) and the presets the benchmarks use.

``qwen35-0.8b`` and ``qwen36-35b-a3b`` restate ModelConfig::qwen35_0_8b and
ModelConfig::qwen36_35b_a3b (src/spec.rs:121-183). ``tiny`` and ``qwen35-2b``
are the shapes named by the benchmark configurations; ``mini-moe`` and
``tiny-moe`` are reduced MoE shapes on the same code paths, sized so the CPU
restatement checks them in seconds.
"""
from __future__ import annotations

import ctypes

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


class CConfig(ctypes.Structure):
    """Mirror of ``cq35_config`` in include/cq35.h."""
    _fields_ = FIELDS


def _dense(**kw):
    base = dict(moe=0, eps=1e-6, theta=10_000_000.0, experts=0, top_k=0,
                shared_intermediate=0, full_interval=4, tied=0)
    base.update(kw)
    return base


def _moe(**kw):
    base = dict(moe=1, eps=1e-6, theta=10_000_000.0, full_interval=4, tied=0)
    base.update(kw)
    return base


PRESETS = {
    # The benchmark's CPU-runnable tiny case: 4 layers (3 DeltaNet + 1 gated attention), hidden
    # 256, DeltaNet 4 QK / 8 V heads of dim 32, attention 4 Q / 1 KV heads of
    # dim 64 (rotary 16 = head_dim/4, the Qwen3.5 partial-rotary ratio), FFN
    # 768, vocab 4096.
    "tiny": _dense(vocab=4096, hidden=256, intermediate=768, layers=4, q_heads=4,
                   kv_heads=1, head_dim=64, rope_dim=16, key_heads=4, key_dim=32,
                   value_heads=8, value_dim=32),
    # src/spec.rs:121-151
    "qwen35-0.8b": _dense(vocab=248_320, hidden=1024, intermediate=3584, layers=24,
                          q_heads=8, kv_heads=2, head_dim=256, rope_dim=64, key_heads=16,
                          key_dim=128, value_heads=16, value_dim=128, tied=1),
    # The benchmark's 2B-shaped dense case
    "qwen35-2b": _dense(vocab=248_320, hidden=2048, intermediate=6144, layers=24,
                        q_heads=8, kv_heads=2, head_dim=256, rope_dim=64, key_heads=16,
                        key_dim=128, value_heads=32, value_dim=128, tied=1),
    # src/spec.rs:153-183
    "qwen36-35b-a3b": _moe(vocab=248_320, hidden=2048, intermediate=512, layers=40,
                           q_heads=16, kv_heads=2, head_dim=256, rope_dim=64, experts=256,
                           top_k=8, shared_intermediate=512, key_heads=16, key_dim=128,
                           value_heads=32, value_dim=128),
    # Reduced dense shape on the key_dim-128 paths (batched prefill); the FFN
    # width leaves a partial last round of 256-lane pairs.
    "mini": _dense(vocab=8192, hidden=512, intermediate=1408, layers=4, q_heads=4,
                   kv_heads=2, head_dim=256, rope_dim=64, key_heads=2, key_dim=128,
                   value_heads=4, value_dim=128),
    # Reduced shapes on the MoE code paths.
    "mini-moe": _moe(vocab=8192, hidden=512, intermediate=128, layers=4, q_heads=4,
                     kv_heads=2, head_dim=256, rope_dim=64, experts=32, top_k=8,
                     shared_intermediate=256, key_heads=2, key_dim=128, value_heads=4,
                     value_dim=128),
    "tiny-moe": _moe(vocab=4096, hidden=256, intermediate=64, layers=4, q_heads=4,
                     kv_heads=1, head_dim=64, rope_dim=16, experts=16, top_k=4,
                     shared_intermediate=128, key_heads=4, key_dim=32, value_heads=8,
                     value_dim=32),
}


def preset(name: str) -> dict:
    if name not in PRESETS:
        raise KeyError(f"unknown preset {name!r}; known: {sorted(PRESETS)}")
    return dict(PRESETS[name])


def to_c(cfg: dict) -> CConfig:
    c = CConfig()
    for name, _ in FIELDS:
        setattr(c, name, cfg[name])
    return c


def from_c(c: CConfig) -> dict:
    out = {name: getattr(c, name) for name, _ in FIELDS}
    out["eps"] = float(c.eps)
    out["theta"] = float(c.theta)
    return out


def derived(cfg: dict) -> dict:
    """Derived sizes (src/spec.rs:293-362)."""
    ks = cfg["key_heads"] * cfg["key_dim"]
    vs = cfg["value_heads"] * cfg["value_dim"]
    qkv = 2 * ks + vs
    return dict(
        key_size=ks, value_size=vs, qkv=qkv, recurrent=vs * cfg["key_dim"], conv=3 * qkv,
        kvs=cfg["kv_heads"] * cfg["head_dim"], query_size=cfg["q_heads"] * cfg["head_dim"],
        full_layers=[l for l in range(cfg["layers"]) if (l + 1) % cfg["full_interval"] == 0],
    )


def is_full(cfg: dict, layer: int) -> bool:
    return (layer + 1) % cfg["full_interval"] == 0


def bytes_per_token(cfg: dict, context: int) -> dict:
    """Algorithmic HBM bytes of one batch-1 decode step at `context` cached
    positions: weights touched (routed experts only for MoE), KV read for
    context+1 positions, DeltaNet state read+write (BF16) and the convolution
    history (read 3 slots, write 1)."""
    d = derived(cfg)
    H, I, V = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
    full = len(d["full_layers"])
    lin = cfg["layers"] - full
    w = H * 2  # embedding row
    w_lin = ((d["qkv"] + d["value_size"] + 2 * cfg["value_heads"]) * H * 2
             + H * d["value_size"] * 2
             + (2 * H + 2 * cfg["value_heads"] + cfg["value_dim"] + 4 * d["qkv"]) * 4)
    w_full = ((2 * d["query_size"] + 2 * d["kvs"]) * H * 2 + H * d["query_size"] * 2
              + (2 * H + 2 * cfg["head_dim"]) * 4)
    if cfg["moe"]:
        SI = cfg["shared_intermediate"]
        w_ffn = (cfg["top_k"] * 3 * I * H * 2 + 3 * SI * H * 2
                 + (cfg["experts"] + 1) * H * 4)
    else:
        w_ffn = 3 * I * H * 2
    w += lin * w_lin + full * w_full + cfg["layers"] * w_ffn
    w += H * 4 + V * H * 2  # final norm + vocabulary head
    kv = full * (context + 1) * 2 * d["kvs"] * 2
    state = lin * (2 * d["recurrent"] * 2 + 4 * d["qkv"] * 2)
    return dict(weights=w, kv=kv, state=state, total=w + kv + state)

"""GGUF version-3 writer for the loader tests (test infrastructure).

Layout (the published GGUF format, as the reference's parser reads it,
src/checkpoint.rs:1181-1261): magic "GGUF", version 3, tensor count and
metadata count (u64), metadata (key string, u32 type, value), tensor infos
(name, u32 dimension count, u64 dimensions innermost first, u32 ggml type,
u64 offset relative to the aligned data start), then the payloads.

`reference_specs` restates the reference's tensor inventory
(src/spec.rs:443-712: GGUF name, shape outermost first, dtype) independently
of the library's own table, so the tests pin the library's names to it.
"""
from __future__ import annotations

import struct

import numpy as np

MAGIC = 0x46554747
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
GGML_F32, GGML_F16, GGML_BF16 = 0, 1, 30


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    fmt = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}[t]
    return struct.pack(fmt, v)


def write(path, metadata, tensors, alignment=32, version=3, magic=MAGIC, truncate_data=False,
          offsets=None):
    """metadata: [(key, type, value)]; tensors: [(name, dims outermost first,
    ggml type, payload bytes)]. offsets overrides the relative offsets."""
    head = struct.pack("<IIQQ", magic, version, len(tensors), len(metadata))
    for key, t, v in metadata:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    rel, pos = [], 0
    for _, _, _, payload in tensors:
        rel.append(pos)
        pos += (len(payload) + alignment - 1) // alignment * alignment
    if offsets is not None:
        rel = offsets
    for (name, dims, gtype, _), off in zip(tensors, rel):
        head += _str(name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in reversed(dims))
        head += struct.pack("<IQ", gtype, off)
    start = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * (start - len(head)))
        if truncate_data:
            return
        end = 0
        for (_, _, _, payload), off in zip(tensors, rel):
            f.seek(start + off)
            f.write(payload)
            end = max(end, start + off + len(payload))
        f.truncate(end)


def reference_specs(cfg: dict):
    """[(gguf name, shape, dtype)] in weight_specs order (src/spec.rs:443-712)."""
    H, V = cfg["hidden"], cfg["vocab"]
    qs = cfg["q_heads"] * cfg["head_dim"]
    kvs = cfg["kv_heads"] * cfg["head_dim"]
    ks = cfg["key_heads"] * cfg["key_dim"]
    inner = cfg["value_heads"] * cfg["value_dim"]
    qkv = 2 * ks + inner
    rank = cfg["value_heads"]
    out = [("token_embd.weight", [V, H], "bf16")]
    for l in range(cfg["layers"]):
        b = f"blk.{l}."
        out.append((b + "attn_norm.weight", [H], "f32"))
        if (l + 1) % cfg["full_interval"] == 0:
            out += [(b + "attn_q.weight", [2 * qs, H], "bf16"), (b + "attn_k.weight", [kvs, H], "bf16"),
                    (b + "attn_v.weight", [kvs, H], "bf16"), (b + "attn_output.weight", [H, qs], "bf16"),
                    (b + "attn_q_norm.weight", [cfg["head_dim"]], "f32"),
                    (b + "attn_k_norm.weight", [cfg["head_dim"]], "f32")]
        else:
            out += [(b + "attn_qkv.weight", [qkv, H], "bf16"), (b + "attn_gate.weight", [inner, H], "bf16"),
                    (b + "ssm_alpha.weight", [rank, H], "bf16"), (b + "ssm_beta.weight", [rank, H], "bf16"),
                    (b + "ssm_dt.bias", [rank], "f32"), (b + "ssm_a", [rank], "f32"),
                    (b + "ssm_norm.weight", [cfg["value_dim"]], "f32"),
                    (b + "ssm_out.weight", [H, inner], "bf16"), (b + "ssm_conv1d.weight", [qkv, 4], "f32")]
        out.append((b + "post_attention_norm.weight", [H], "f32"))
        I = cfg["intermediate"]
        if not cfg["moe"]:
            out += [(b + "ffn_gate.weight", [I, H], "bf16"), (b + "ffn_up.weight", [I, H], "bf16"),
                    (b + "ffn_down.weight", [H, I], "bf16")]
        else:
            E = cfg["experts"]
            out += [(b + "ffn_gate_inp.weight", [E, H], "f32"),
                    (b + "ffn_gate_exps.weight", [E, I, H], "bf16"),
                    (b + "ffn_up_exps.weight", [E, I, H], "bf16"),
                    (b + "ffn_down_exps.weight", [E, H, I], "bf16")]
        if cfg["moe"] and cfg["shared_intermediate"]:
            SI = cfg["shared_intermediate"]
            out += [(b + "ffn_gate_inp_shexp.weight", [1, H], "f32"),
                    (b + "ffn_gate_shexp.weight", [SI, H], "bf16"),
                    (b + "ffn_up_shexp.weight", [SI, H], "bf16"),
                    (b + "ffn_down_shexp.weight", [H, SI], "bf16")]
    out.append(("output_norm.weight", [H], "f32"))
    out.append(("token_embd.weight" if cfg["tied"] else "output.weight", [V, H], "bf16"))
    return out


def metadata(cfg: dict, vocab_key=True, nextn=0, arch=None):
    """The architecture-scoped keys parse_gguf_model_config reads
    (src/checkpoint.rs:422-639), as real Qwen3.5/3.6 GGUFs carry them."""
    arch = arch or ("qwen35moe" if cfg["moe"] else "qwen35")
    a = arch + "."
    md = [("general.architecture", STRING, arch), ("general.name", STRING, "synthetic"),
          (a + "embedding_length", U32, cfg["hidden"]),
          (a + "block_count", U32, cfg["layers"] + nextn),
          (a + "attention.head_count", U32, cfg["q_heads"]),
          (a + "attention.head_count_kv", U32, cfg["kv_heads"]),
          (a + "attention.key_length", U32, cfg["head_dim"]),
          (a + "context_length", U32, 262144),
          (a + "attention.layer_norm_rms_epsilon", F32, cfg["eps"]),
          (a + "rope.freq_base", F32, cfg["theta"]),
          (a + "rope.dimension_count", U32, cfg["rope_dim"]),
          (a + "rope.dimension_sections", ARRAY, (I32, [11, 11, 10, 0])),
          (a + "full_attention_interval", U32, cfg["full_interval"]),
          (a + "ssm.conv_kernel", U32, 4),
          (a + "ssm.state_size", U32, cfg["key_dim"]),
          (a + "ssm.group_count", U32, cfg["key_heads"]),
          (a + "ssm.time_step_rank", U32, cfg["value_heads"]),
          (a + "ssm.inner_size", U32, cfg["value_heads"] * cfg["value_dim"])]
    if vocab_key:
        md.append((a + "vocab_size", U32, cfg["vocab"]))
    else:
        md.append(("tokenizer.ggml.tokens", ARRAY, (STRING, [f"t{i}" for i in range(cfg["vocab"])])))
    if nextn:
        md.append((a + "nextn_predict_layers", U32, nextn))
    if cfg["moe"]:
        md += [(a + "expert_feed_forward_length", U32, cfg["intermediate"]),
               (a + "expert_count", U32, cfg["experts"]),
               (a + "expert_used_count", U32, cfg["top_k"]),
               (a + "expert_shared_feed_forward_length", U32, cfg["shared_intermediate"])]
    else:
        md.append((a + "feed_forward_length", U32, cfg["intermediate"]))
    return md


def tensors_for(cfg: dict, arrays=None):
    """Tensor list for `cfg`; payloads from `arrays` (weight_specs order, the
    tied head omitted) or zero bytes of the right size."""
    out, seen = [], set()
    for i, (name, shape, dtype) in enumerate(reference_specs(cfg)):
        if name in seen:
            continue  # the tied head is the embedding tensor itself
        seen.add(name)
        size = int(np.prod(shape)) * (2 if dtype == "bf16" else 4)
        if arrays is None:
            payload = bytes(size)
        else:
            payload = np.ascontiguousarray(arrays[i]).tobytes()
            assert len(payload) == size, (name, len(payload), size)
        out.append((name, shape, GGML_BF16 if dtype == "bf16" else GGML_F32, payload))
    return out

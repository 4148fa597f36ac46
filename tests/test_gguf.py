"""GGUF checkpoints on the CPU (no GPU needed): configuration from metadata,
tensor inventory / shape / dtype / range validation, shard sets and
directories, next-token layers and the tied head. Mirrors the reference's
loader tests (src/checkpoint.rs:1471-1637) and its validation rules
(validate_files, tensor_view: checkpoint.rs:659-820). The files come from
`gguf_writer`, whose tensor table restates src/spec.rs:443-712 on its own."""
import os

import numpy as np
import pytest

import cq35
import cq35.config as cc
import gguf_writer as gw

PRESETS = ["tiny", "tiny-moe", "mini", "mini-moe", "qwen36-35b-a3b"]


def full_file(path, cfg, **kw):
    gw.write(path, gw.metadata(cfg, **{k: v for k, v in kw.items() if k in ("vocab_key", "nextn", "arch")}),
             gw.tensors_for(cfg), truncate_data=kw.get("truncate_data", False))


def error_text(fn, *a):
    with pytest.raises(cq35.CQ35Error) as e:
        fn(*a)
    return str(e.value)


@pytest.mark.parametrize("name", PRESETS)
def test_tensor_names_match_reference_spec(name):
    cfg = cc.preset(name)
    specs = gw.reference_specs(cfg)
    assert len(specs) == cq35.weight_count(cfg)
    for i, (gname, shape, dtype) in enumerate(specs):
        assert cq35.gguf_tensor_name(cfg, i) == gname
        info = cq35.weight_info(cfg, i)
        assert info.rows * info.cols == int(np.prod(shape)), gname
        assert info.dtype == (0 if dtype == "bf16" else 1), gname


@pytest.mark.parametrize("name", PRESETS)
def test_config_round_trip(tmp_path, name):
    cfg = cc.preset(name)
    p = str(tmp_path / "m.gguf")
    # headers only: the configuration never reads the payloads
    full_file(p, cfg, truncate_data=True)
    got = cq35.gguf_config(p)
    for k, v in cfg.items():
        assert got[k] == pytest.approx(v) if isinstance(v, float) else got[k] == v, k


def test_vocabulary_from_tokenizer_tokens(tmp_path):
    cfg = cc.preset("tiny-moe")
    p = str(tmp_path / "m.gguf")
    full_file(p, cfg, vocab_key=False, truncate_data=True)
    assert cq35.gguf_config(p)["vocab"] == cfg["vocab"]


def test_complete_file_validates(tmp_path):
    cfg = cc.preset("mini-moe")
    p = str(tmp_path / "m.gguf")
    full_file(p, cfg)
    cq35.gguf_validate(p)
    cq35.gguf_validate(p, cfg)
    other = dict(cfg, top_k=4)
    assert "different configuration" in error_text(cq35.gguf_validate, p, other)


def test_tied_head_follows_output_tensor(tmp_path):
    cfg = dict(cc.preset("mini"), tied=1)
    p = str(tmp_path / "tied.gguf")
    full_file(p, cfg)
    assert cq35.gguf_config(p)["tied"] == 1
    cq35.gguf_validate(p)
    untied = dict(cfg, tied=0)
    q = str(tmp_path / "untied.gguf")
    gw.write(q, gw.metadata(untied), gw.tensors_for(untied))
    assert cq35.gguf_config(q)["tied"] == 0
    cq35.gguf_validate(q)


def test_next_token_layers_are_ignored(tmp_path):
    cfg = cc.preset("tiny-moe")
    p = str(tmp_path / "m.gguf")
    extra = [(f"blk.{cfg['layers']}.nextn.eh_proj.weight", [cfg["hidden"], 2 * cfg["hidden"]],
              gw.GGML_BF16, bytes(2 * 2 * cfg["hidden"] * cfg["hidden"]))]
    gw.write(p, gw.metadata(cfg, nextn=1), gw.tensors_for(cfg) + extra)
    got = cq35.gguf_config(p)
    assert got["layers"] == cfg["layers"]
    cq35.gguf_validate(p)
    # without the metadata key the same tensor is unexpected
    q = str(tmp_path / "n.gguf")
    gw.write(q, gw.metadata(cfg), gw.tensors_for(cfg) + extra)
    assert "unexpected" in error_text(cq35.gguf_validate, q)


def test_shard_set_and_directory(tmp_path):
    cfg = cc.preset("tiny-moe")
    tensors = gw.tensors_for(cfg)
    parts = [tensors[0::3], tensors[1::3], tensors[2::3]]
    d = tmp_path / "shards"
    d.mkdir()
    names = [str(d / f"model-BF16-0000{i + 1}-of-00003.gguf") for i in range(3)]
    for i, (n, part) in enumerate(zip(names, parts)):
        gw.write(n, gw.metadata(cfg) if i == 0 else [("general.architecture", gw.STRING, "qwen35moe")], part)
    (d / "tokenizer.json").write_text("{}")
    for member in names:  # any member names the whole set
        assert cq35.gguf_config(member) == cq35.gguf_config(names[0])
        cq35.gguf_validate(member)
    cq35.gguf_validate(str(d))
    assert cq35.gguf_config(str(d))["experts"] == cfg["experts"]
    os.remove(names[2])
    assert "cannot" in error_text(cq35.gguf_validate, names[0])


def test_duplicate_tensor_across_shards(tmp_path):
    cfg = cc.preset("tiny-moe")
    tensors = gw.tensors_for(cfg)
    d = tmp_path / "dup"
    d.mkdir()
    gw.write(str(d / "a-00001-of-00002.gguf"), gw.metadata(cfg), tensors)
    gw.write(str(d / "a-00002-of-00002.gguf"), [], tensors[:1])
    assert "duplicate" in error_text(cq35.gguf_validate, str(d / "a-00001-of-00002.gguf"))


@pytest.mark.parametrize("case", ["magic", "version", "missing", "unexpected", "shape", "dtype", "f16",
                                  "range", "overlap", "misaligned", "arch", "key", "conv"])
def test_rejections(tmp_path, case):
    cfg = cc.preset("tiny-moe")
    p = str(tmp_path / "bad.gguf")
    md, tensors, kw = gw.metadata(cfg), gw.tensors_for(cfg), {}
    if case == "magic":
        kw["magic"] = 0x46554748
    elif case == "version":
        kw["version"] = 2
    elif case == "missing":
        tensors = [t for t in tensors if t[0] != "blk.1.ssm_a"]
    elif case == "unexpected":
        tensors = tensors + [("blk.0.extra.weight", [4], gw.GGML_F32, bytes(16))]
    elif case == "shape":
        tensors = [(n, [s[1], s[0]] if n == "blk.0.attn_qkv.weight" else s, t, b) for n, s, t, b in tensors]
    elif case == "dtype":
        tensors = [(n, s, gw.GGML_F32 if n == "blk.0.attn_gate.weight" else t,
                    b + b if n == "blk.0.attn_gate.weight" else b) for n, s, t, b in tensors]
    elif case == "f16":
        tensors = [(n, s, gw.GGML_F16 if n == "blk.0.attn_gate.weight" else t, b) for n, s, t, b in tensors]
    elif case == "range":
        kw["truncate_data"] = True
    elif case == "overlap":
        kw["offsets"] = [0] * len(tensors)
    elif case == "misaligned":
        kw["offsets"] = [0] + [1] * (len(tensors) - 1)
    elif case == "arch":
        md = [(k, t, "qwen3") if k == "general.architecture" else (k, t, v) for k, t, v in md]
    elif case == "key":
        md = [m for m in md if not m[0].endswith(".ssm.state_size")]
    elif case == "conv":
        md = [(k, t, 3) if k.endswith(".ssm.conv_kernel") else (k, t, v) for k, t, v in md]
    gw.write(p, md, tensors, **kw)
    text = error_text(cq35.gguf_validate, p)
    expect = {"magic": "magic", "version": "version 3", "missing": "missing (blk.1.ssm_a)",
              "unexpected": "unexpected (blk.0.extra.weight)", "shape": "has shape",
              "dtype": "has dtype", "f16": "BF16/F32", "range": "exceeds", "overlap": "overlap",
              "misaligned": "not aligned", "arch": "outside this build", "key": "ssm.state_size",
              "conv": "four convolution taps"}[case]
    assert expect in text, text

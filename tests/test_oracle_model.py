"""CPU checks of the restated token loop: the weight ABI and presets against
src/spec.rs, the byte model, and the whole decode step against a float64
textbook formulation (semantics pinned to within BF16 activation noise, with
planted mistakes shown to exceed the tolerance)."""
import numpy as np
import pytest

import cq35.config as cc
from textbook import Textbook


def test_weight_abi_counts(oracle):
    # per-layer group sizes of the generated entry (src/qwen/qwen35.rs:1489-1497)
    moe = cc.preset("qwen36-35b-a3b")
    assert len(oracle.weight_specs(moe)) == 1 + 30 * 19 + 10 * 16 + 2 == 733
    dense = cc.preset("qwen35-0.8b")
    assert len(oracle.weight_specs(dense)) == 1 + 18 * 14 + 6 * 11 + 2
    specs = oracle.weight_specs(moe)
    # layer 0 (linear): attn_norm, qkv, z, alpha, beta, dt, a, ssm_norm, out, conv, post, router...
    assert [s[:3] for s in specs[1:11]] == [
        ("f32", 2048, 1), ("bf16", 8192, 2048), ("bf16", 4096, 2048), ("bf16", 32, 2048),
        ("bf16", 32, 2048), ("f32", 32, 1), ("f32", 32, 1), ("f32", 128, 1), ("bf16", 2048, 4096),
        ("f32", 8192, 4)]
    assert [s[:3] for s in specs[11:20]] == [
        ("f32", 2048, 1), ("f32", 256, 2048), ("bf16", 256 * 512, 2048), ("bf16", 256 * 512, 2048),
        ("bf16", 256 * 2048, 512), ("f32", 1, 2048), ("bf16", 512, 2048), ("bf16", 512, 2048),
        ("bf16", 2048, 512)]
    # layer 3 is the first full-attention layer: q (2*Q*HD), k, v, o, q_norm, k_norm
    full0 = 1 + 3 * 19
    assert [s[:3] for s in specs[full0:full0 + 8]] == [
        ("f32", 2048, 1), ("bf16", 8192, 2048), ("bf16", 512, 2048), ("bf16", 512, 2048),
        ("bf16", 2048, 4096), ("f32", 256, 1), ("f32", 256, 1), ("f32", 2048, 1)]
    assert specs[-1][:3] == ("bf16", 248320, 2048) and specs[-2][:3] == ("f32", 2048, 1)


def test_presets_match_reference_spec():
    # ModelConfig::qwen35_0_8b / qwen36_35b_a3b (src/spec.rs:121-183)
    a = cc.preset("qwen35-0.8b")
    assert (a["vocab"], a["hidden"], a["intermediate"], a["layers"], a["q_heads"], a["kv_heads"],
            a["head_dim"], a["rope_dim"], a["key_heads"], a["key_dim"],
            a["value_heads"] * a["value_dim"], a["value_heads"], a["tied"]) == \
        (248_320, 1024, 3584, 24, 8, 2, 256, 64, 16, 128, 2048, 16, 1)
    b = cc.preset("qwen36-35b-a3b")
    assert (b["vocab"], b["hidden"], b["intermediate"], b["layers"], b["q_heads"], b["kv_heads"],
            b["head_dim"], b["rope_dim"], b["experts"], b["top_k"], b["shared_intermediate"],
            b["key_heads"], b["key_dim"], b["value_heads"] * b["value_dim"], b["value_heads"],
            b["tied"]) == \
        (248_320, 2048, 512, 40, 16, 2, 256, 64, 256, 8, 512, 16, 128, 4096, 32, 0)
    assert np.float32(b["eps"]) == np.float32(1e-6) and b["theta"] == 1e7


def test_bytes_per_token_model():
    b = cc.bytes_per_token(cc.preset("qwen36-35b-a3b"), 1024)
    assert abs(b["weights"] / 1e9 - 5.937) < 0.01
    assert abs(b["total"] / 1e9 - 6.02) < 0.01


def run_oracle(oracle, cfg, seed, tokens, steps, multi=False):
    weights = oracle.synthetic_weights(cfg, seed)
    model = oracle.Model(cfg, weights)
    s = model.session(len(tokens) + steps + 1)
    out = []
    if multi:
        nxt, logits = s.step(tokens, 0)
        out.append(logits)
        pos = len(tokens)
    else:
        for i, t in enumerate(tokens):
            nxt, logits = s.step([t], i)
        out.append(logits)
        pos = len(tokens)
    for _ in range(steps):
        nxt, logits = s.step([nxt], pos)
        pos += 1
        out.append(logits)
    return weights, out, s


def textbook_logits(cfg, weights, tokens, steps, oracle_logits, key_head=None):
    tb = Textbook(cfg, weights, **({"key_head": key_head} if key_head else {}))
    res = []
    for i, t in enumerate(tokens):
        logits = tb.step(t, i)
    res.append(logits)
    pos = len(tokens)
    for k in range(steps):
        # feed the restatement's greedy tokens so both see the same inputs
        nxt = int(np.argmax(oracle_logits[k].view(np.uint16)))
        bits = oracle_logits[k]
        f = (bits.astype(np.uint32) << 16).view(np.float32)
        nxt = int(np.argmax(f))
        logits = tb.step(nxt, pos)
        pos += 1
        res.append(logits)
    return res


def discrepancy(oracle_logits, tb_logits):
    """Worst relative RMS error of the logits over the steps (BF16 activation
    rounding alone gives a few percent)."""
    worst = 0.0
    for o, t in zip(oracle_logits, tb_logits):
        f = (o.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        worst = max(worst, float(np.sqrt(np.mean((f - t) ** 2)) / np.std(t)))
    return worst


@pytest.mark.parametrize("name", ["tiny", "tiny-moe", "mini-moe"])
def test_restatement_matches_textbook(oracle, name):
    cfg = cc.preset(name)
    rng = np.random.default_rng(11)
    tokens = rng.integers(0, cfg["vocab"], 6).tolist()
    weights, ol, _ = run_oracle(oracle, cfg, 5, tokens, 4)
    tl = textbook_logits(cfg, weights, tokens, 4, ol)
    d = discrepancy(ol, tl)
    assert d < 0.15, d
    # planted mistake in the checker's semantics: value head h reading key
    # head h // (VH/KH) (the HF layout) instead of the GGUF h % KH
    if cfg["value_heads"] != cfg["key_heads"]:
        r = cfg["value_heads"] // cfg["key_heads"]
        tl_bad = textbook_logits(cfg, weights, tokens, 4, ol, key_head=lambda h, KH, VH: h // r)
        assert discrepancy(ol, tl_bad) > 0.6


def test_multi_token_call_keeps_f32_state(oracle):
    """A multi-token call carries the DeltaNet state in F32 between tokens
    (token fold, qwen35.rs:1395-1465 with import/persist); it stays within
    BF16 noise of the per-token calls and of the textbook."""
    cfg = cc.preset("tiny")
    tokens = np.random.default_rng(2).integers(0, cfg["vocab"], 16).tolist()
    w, multi, _ = run_oracle(oracle, cfg, 9, tokens, 0, multi=True)
    _, single, _ = run_oracle(oracle, cfg, 9, tokens, 0, multi=False)
    tl = textbook_logits(cfg, w, tokens, 0, multi)
    assert discrepancy(multi, tl) < 0.15
    assert discrepancy(single, tl) < 0.15


@pytest.mark.parametrize("name", ["mini", "mini-moe"])
def test_batched_prefill_matches_textbook(oracle, name):
    """A multi-token call at key_dim 128 takes the batched prefill (layer-major,
    B256 projections, F32 scan state); its logits and the decode steps after
    it stay within BF16 noise of the textbook, and a planted key-head mistake
    in the textbook is detected."""
    cfg = cc.preset(name)
    tokens = np.random.default_rng(4).integers(0, cfg["vocab"], 12).tolist()
    w, batched, s = run_oracle(oracle, cfg, 7, tokens, 3, multi=True)
    tl = textbook_logits(cfg, w, tokens, 3, batched)
    assert discrepancy(batched, tl) < 0.15
    r = cfg["value_heads"] // cfg["key_heads"]
    bad = textbook_logits(cfg, w, tokens, 3, batched, key_head=lambda h, KH, VH: h // r)
    assert discrepancy(batched, bad) > 0.6


def test_batched_prefill_differs_from_token_fold_only_by_order(oracle):
    """The batched path's B256 projections round differently from the decode
    S256/S32 ones, so a batched prompt and the same prompt appended token by
    token agree to BF16 noise but not bit for bit."""
    cfg = cc.preset("mini-moe")
    tokens = np.random.default_rng(8).integers(0, cfg["vocab"], 10).tolist()
    _, batched, sb = run_oracle(oracle, cfg, 3, tokens, 0, multi=True)
    _, single, ss = run_oracle(oracle, cfg, 3, tokens, 0, multi=False)
    fb = oracle.bf16_to_f32(batched[0]).astype(np.float64)
    fs = oracle.bf16_to_f32(single[0]).astype(np.float64)
    rel = float(np.sqrt(np.mean((fb - fs) ** 2)) / np.std(fs))
    assert 0 < rel < 0.1, rel

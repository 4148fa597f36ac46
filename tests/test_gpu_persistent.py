"""The persistent one-launch decode steps against the per-kernel launch
sequence and the CPU restatement: greedy tokens, BF16 logits and the whole
session state bit-exact, on the reduced MoE shapes, the full 35B-A3B
shape and the dense shapes (tiny, mini, 0.8B, 2B)
(src/qwen/qwen35.rs:1395-1465 is the step both implement)."""
import numpy as np
import pytest

import cq35
import cq35.config as cc

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def run(model, prompt, steps, persistent, capacity):
    s = model.session(capacity)
    s.set_persistent(persistent)
    assert s.persistent == persistent
    calls = []
    for t in prompt:
        logits, tok = s.step_raw([t])
        calls.append((tok, logits))
    tok = calls[-1][0]
    for _ in range(steps):
        logits, tok = s.step_raw([tok])
        calls.append((tok, logits))
    return s, calls


@pytest.mark.parametrize("name", ["tiny-moe", "mini-moe"])
def test_persistent_is_the_default_decode_path(name):
    cfg = cc.preset(name)
    m = cq35.Model.synthetic(cfg, seed=1)
    s = m.session(32)
    assert s.persistent, f"{name}: the persistent kernel should cover this shape"
    # dense shapes: persistent up to 8064 cached positions, per-kernel beyond
    dense = cq35.Model.synthetic(cc.preset("tiny"), seed=1)
    assert dense.session(8).persistent
    assert dense.session(8064).persistent
    long = dense.session(8065)
    assert not long.persistent
    with pytest.raises(cq35.CQ35Error):
        long.set_persistent(True)


@pytest.mark.parametrize("name,prompt_len,steps", [("mini-moe", 40, 40), ("qwen36-35b-a3b", 20, 12)])
def test_persistent_matches_per_kernel_path(name, prompt_len, steps):
    cfg = cc.preset(name)
    say("persistent vs per-kernel", name, "prompt", prompt_len, "steps", steps)
    m = cq35.Model.synthetic(cfg, seed=5)
    prompt = np.random.default_rng(41).integers(0, cfg["vocab"], prompt_len).tolist()
    cap = prompt_len + steps + 4
    sa, ca = run(m, prompt, steps, True, cap)
    say("  persistent done")
    sb, cb = run(m, prompt, steps, False, cap)
    say("  per-kernel done")
    for i, ((ta, la), (tb, lb)) in enumerate(zip(ca, cb)):
        assert ta == tb, f"{name}: token differs at call {i}: {ta} vs {tb}"
        assert np.array_equal(la, lb), f"{name}: logits differ at call {i}"
    assert np.array_equal(sa.export_state(0), sb.export_state(0)), f"{name}: cache state differs"


@pytest.mark.parametrize("name,prompt_len,steps", [("tiny", 24, 40), ("mini", 20, 24)])
def test_dense_persistent_matches_per_kernel_and_oracle(oracle, name, prompt_len, steps):
    cfg = cc.preset(name)
    say("dense persistent vs per-kernel vs oracle", name, "prompt", prompt_len, "steps", steps)
    m = cq35.Model.synthetic(cfg, seed=5)
    prompt = np.random.default_rng(43).integers(0, cfg["vocab"], prompt_len).tolist()
    cap = prompt_len + steps + 4
    sa, ca = run(m, prompt, steps, True, cap)
    say("  persistent done")
    sb, cb = run(m, prompt, steps, False, cap)
    say("  per-kernel done")
    om = oracle.Model(cfg, oracle.synthetic_weights(cfg, 5))
    os_ = om.session(cap)
    co = []
    for i, t in enumerate(prompt):
        tok, logits = os_.step([t], i)
        co.append((tok, logits))
    tok = co[-1][0]
    for i in range(steps):
        tok, logits = os_.step([tok], prompt_len + i)
        co.append((tok, logits))
    say("  oracle done")
    for i, ((ta, la), (tb, lb), (to, lo)) in enumerate(zip(ca, cb, co)):
        assert ta == tb == to, f"{name}: token differs at call {i}: {ta} {tb} {to}"
        assert np.array_equal(la, lb), f"{name}: persistent/per-kernel logits differ at call {i}"
        assert np.array_equal(la, lo), f"{name}: persistent/oracle logits differ at call {i}"
    want = os_.cache()
    assert np.array_equal(sa.export_state(0), want), f"{name}: persistent state differs"
    assert np.array_equal(sb.export_state(0), want), f"{name}: per-kernel state differs"


@pytest.mark.parametrize("name,prompt_len,steps", [("qwen35-0.8b", 12, 16), ("qwen35-2b", 12, 16)])
def test_dense_persistent_matches_per_kernel_full_shapes(name, prompt_len, steps):
    cfg = cc.preset(name)
    say("dense persistent vs per-kernel", name, "prompt", prompt_len, "steps", steps)
    m = cq35.Model.synthetic(cfg, seed=5)
    prompt = np.random.default_rng(47).integers(0, cfg["vocab"], prompt_len).tolist()
    cap = prompt_len + steps + 4
    sa, ca = run(m, prompt, steps, True, cap)
    say("  persistent done")
    sb, cb = run(m, prompt, steps, False, cap)
    say("  per-kernel done")
    for i, ((ta, la), (tb, lb)) in enumerate(zip(ca, cb)):
        assert ta == tb, f"{name}: token differs at call {i}: {ta} vs {tb}"
        assert np.array_equal(la, lb), f"{name}: logits differ at call {i}"
    assert np.array_equal(sa.export_state(0), sb.export_state(0)), f"{name}: cache state differs"

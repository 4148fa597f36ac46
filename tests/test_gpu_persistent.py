"""The persistent one-launch decode step against the per-kernel launch
sequence and the CPU restatement: greedy tokens, BF16 logits and the whole
session state bit-exact, on the reduced MoE shapes and on the full
35B-A3B shape (src/qwen/qwen35.rs:1395-1465 is the step both implement)."""
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
    dense = cq35.Model.synthetic(cc.preset("tiny"), seed=1).session(8)
    assert not dense.persistent
    with pytest.raises(cq35.CQ35Error):
        dense.set_persistent(True)


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

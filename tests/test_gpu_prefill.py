"""The batched prefill (multi-token calls at key_dim 128; text-dispatch ->
text-batch, src/qwen/prefill.rs:36-653) against the CPU restatement on an
MI355X: greedy token, BF16 logits and the whole session state bit-exact after
the batched call and over the decode steps that follow it, for a dense and a
MoE shape, calls spanning two 256-token chunks (dense and MoE), and a call
that starts after earlier tokens (convolution taps from the cache history)."""
import numpy as np
import pytest

import cq35
import cq35.config as cc

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def check_calls(name, calls):
    for i, (gt, gl, ot, ol) in enumerate(calls):
        assert gt == ot, f"{name}: greedy token differs at call {i}: {gt} vs {ot}"
        assert np.array_equal(gl, ol), f"{name}: logits differ at call {i}"


def run(oracle, name, seed, before, prompt, steps):
    """`before` single-token calls, one batched call of `prompt`, then `steps`
    greedy decode steps, on the GPU and the restatement side by side."""
    cfg = cc.preset(name)
    say("batched prefill", name, "seed", seed, "before", len(before), "prompt", len(prompt),
        "steps", steps)
    gm = cq35.Model.synthetic(cfg, seed=seed)
    om = oracle.Model(cfg, oracle.synthetic_weights(cfg, seed))
    cap = len(before) + len(prompt) + steps + 1
    gs, os_ = gm.session(cap), om.session(cap)
    calls = []
    pos = 0
    for t in before:
        gl, gt = gs.step_raw([t])
        ot, ol = os_.step([t], pos)
        calls.append((gt, gl, ot, ol))
        pos += 1
    gl, gt = gs.step_raw(prompt)
    ot, ol = os_.step(prompt, pos)
    calls.append((gt, gl, ot, ol))
    pos += len(prompt)
    check_calls(name, calls)
    assert np.array_equal(gs.export_state(0), os_.cache()), f"{name}: state after the prefill"
    nxt = gt
    for _ in range(steps):
        gl, gt = gs.step_raw([nxt])
        ot, ol = os_.step([nxt], pos)
        calls.append((gt, gl, ot, ol))
        pos += 1
        nxt = gt
        if gt != ot:
            break
    check_calls(name, calls)
    assert np.array_equal(gs.export_state(0), os_.cache()), f"{name}: state after decoding"
    gm.close()


@pytest.mark.parametrize("name", ["mini", "mini-moe"])
def test_batched_prefill_parity(oracle, name):
    cfg = cc.preset(name)
    prompt = np.random.default_rng(51).integers(0, cfg["vocab"], 37).tolist()
    run(oracle, name, 13, [], prompt, 24)


def test_batched_prefill_after_decoded_tokens(oracle):
    cfg = cc.preset("mini-moe")
    rng = np.random.default_rng(52)
    before = rng.integers(0, cfg["vocab"], 5).tolist()
    prompt = rng.integers(0, cfg["vocab"], 2).tolist()  # shorter than the 3-tap history
    run(oracle, "mini-moe", 14, before, prompt, 4)
    prompt = rng.integers(0, cfg["vocab"], 19).tolist()
    run(oracle, "mini-moe", 15, before, prompt, 4)


def test_batched_prefill_two_chunks(oracle):
    cfg = cc.preset("mini")
    prompt = np.random.default_rng(53).integers(0, cfg["vocab"], 300).tolist()
    run(oracle, "mini", 16, [], prompt, 3)


def test_batched_prefill_two_chunks_moe(oracle):
    """300 MoE tokens: the first 256-token chunk routes about 64 tokens to each
    of mini-moe's 32 experts, so the grouped gate/up runs its per-lane
    epilogues across the 64-token boundary."""
    cfg = cc.preset("mini-moe")
    prompt = np.random.default_rng(54).integers(0, cfg["vocab"], 300).tolist()
    run(oracle, "mini-moe", 17, [], prompt, 3)

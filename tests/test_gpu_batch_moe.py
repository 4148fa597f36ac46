"""The weight-shared batched decode step for MoE sessions (cq35_step_batch on
sessions of one MoE model and capacity: non-expert weights read once per
round, each distinct routed expert once, the shared expert once) against the
same sessions stepped alone (persistent step): greedy tokens, BF16 logits
and every layer's expert ids at every round, the whole state at the end, bit
for bit. Batch sizes that fill and do not fill the 4-token groups, sessions
at different positions, sessions whose attention runs split-K next to
sessions on the single chain, experts shared by several tokens of a round,
and the per-session path (CQ35_BATCH_SHARED=0) as a second reference."""
import os

import numpy as np
import pytest

import cq35
import cq35.config as cc

pytestmark = pytest.mark.gpu

_models = {}


def say(*a):
    print(*a, flush=True)


def model_of(name):
    if name not in _models:
        _models[name] = cq35.Model.synthetic(cc.preset(name), seed=31)
    return _models[name]


def run_batch(model, prompts, splits, rounds, cap):
    group = []
    nxt = []
    for p, sp in zip(prompts, splits):
        s = model.session(cap)
        if sp is not None:
            s.set_attention_split(sp)
        nxt.append(s.append_next_token(p))
        group.append(s)
    calls = []
    for _ in range(rounds):
        nxt, lg = cq35.decode_batch(group, nxt, logits=True)
        calls.append((list(nxt), lg, [s.router_ids() for s in group]))
    return group, calls


@pytest.mark.parametrize("name,B", [("tiny-moe", 2), ("tiny-moe", 7), ("mini-moe", 5), ("mini-moe", 8),
                                    ("mini-moe", 17)])
def test_moe_batch_matches_sessions_alone(name, B):
    cfg = cc.preset(name)
    model = model_of(name)
    rounds, cap = 6, 160
    rng = np.random.default_rng(B)
    prompts = [rng.integers(0, cfg["vocab"], int(rng.integers(2, 120))).tolist() for _ in range(B)]
    # every third session splits its attention above 24 keys (ranges of
    # ceil(T / 128) tiles, then the merge); the rest keep the single chain
    splits = [24 if b % 3 == 1 else None for b in range(B)]
    say("MoE batch", name, B, "prompt lengths", [len(p) for p in prompts])
    group, calls = run_batch(model, prompts, splits, rounds, cap)
    shared = 0
    for b in range(B):
        alone = model.session(cap)
        if splits[b] is not None:
            alone.set_attention_split(splits[b])
        t = alone.append_next_token(prompts[b])
        for r in range(rounds):
            lg, t2 = alone.step_raw([t])
            want_ids = alone.router_ids()
            got_t, got_lg, got_ids = calls[r][0][b], calls[r][1][b], calls[r][2][b]
            assert np.array_equal(got_ids, want_ids), f"{name} B={B} session {b}: expert ids differ at round {r}"
            assert got_t == t2, f"{name} B={B} session {b}: token differs at round {r}"
            assert np.array_equal(got_lg, lg), f"{name} B={B} session {b}: logits differ at round {r}"
            t = t2
        assert np.array_equal(alone.export_state(0), group[b].export_state(0)), f"{name} B={B} session {b}: state"
    # experts chosen by several tokens of one round (the union path) occur
    for r in range(rounds):
        for layer in range(cfg["layers"]):
            chosen = np.concatenate([calls[r][2][b][layer] for b in range(B)])
            shared += len(chosen) - len(np.unique(chosen))
    say(f"  expert selections shared within a round: {shared}")
    if B >= 5:
        assert shared > 0


def test_moe_batch_equals_per_session_path():
    name, B, rounds, cap = "mini-moe", 6, 4, 64
    cfg = cc.preset(name)
    model = model_of(name)
    prompts = [[(11 * b + 5 * i) % cfg["vocab"] for i in range(3 + 4 * b)] for b in range(B)]
    out = {}
    for shared in ("1", "0"):
        os.environ["CQ35_BATCH_SHARED"] = shared
        try:
            group, calls = run_batch(model, prompts, [None] * B, rounds, cap)
            out[shared] = ([c[0] for c in calls], [c[1] for c in calls], [s.export_state(0) for s in group])
        finally:
            os.environ.pop("CQ35_BATCH_SHARED", None)
    assert out["1"][0] == out["0"][0]
    for a, b in zip(out["1"][1], out["0"][1]):
        assert np.array_equal(a, b)
    for a, b in zip(out["1"][2], out["0"][2]):
        assert np.array_equal(a, b)

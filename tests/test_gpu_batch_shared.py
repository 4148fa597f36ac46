"""The weight-shared batched decode step (dense sessions of one model and
capacity stepped by cq35_step_batch: every layer's weights read once for all
the sessions' tokens) against the same sessions stepped alone: greedy
tokens and whole session states bit for bit, for batch sizes that fill and
do not fill the GEMVs' 4-token groups, sessions at different positions,
several rounds, and the per-session overlapped path (CQ35_BATCH_SHARED=0)."""
import os

import numpy as np
import pytest

import cq35
import cq35.config as cc

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def mini():
    cfg = cc.preset("mini")
    return cfg, cq35.Model.synthetic(cfg, seed=12)


@pytest.mark.parametrize("B", [2, 5, 16, 21])
def test_shared_batch_matches_sessions_alone(mini, B):
    cfg, model = mini
    rounds, cap = 5, 48
    rng = np.random.default_rng(B)
    prompts = [rng.integers(0, cfg["vocab"], int(rng.integers(2, 30))).tolist() for _ in range(B)]
    say("shared batch", B, "prompt lengths", [len(p) for p in prompts])
    group = [model.session(cap) for _ in range(B)]
    nxt = [s.append_next_token(p) for s, p in zip(group, prompts)]
    history = [list(nxt)]
    for _ in range(rounds):
        nxt = cq35.decode_batch(group, nxt)
        history.append(list(nxt))
    for b in range(B):
        alone = model.session(cap)
        t = alone.append_next_token(prompts[b])
        assert t == history[0][b]
        for r in range(rounds):
            t = alone.decode_next_token(t)
            assert t == history[r + 1][b], f"B={B} session {b}: token differs at round {r}"
        assert np.array_equal(alone.export_state(0), group[b].export_state(0)), f"B={B} session {b}: state"


def test_shared_batch_equals_overlapped_path(mini):
    cfg, model = mini
    B, rounds, cap = 6, 4, 40
    prompts = [[(13 * b + 7 * i) % cfg["vocab"] for i in range(3 + b)] for b in range(B)]
    out = {}
    for shared in ("1", "0"):
        os.environ["CQ35_BATCH_SHARED"] = shared
        try:
            group = [model.session(cap) for _ in range(B)]
            nxt = [s.append_next_token(p) for s, p in zip(group, prompts)]
            seq = [list(nxt)]
            for _ in range(rounds):
                nxt = cq35.decode_batch(group, nxt)
                seq.append(list(nxt))
            out[shared] = (seq, [s.export_state(0) for s in group])
        finally:
            os.environ.pop("CQ35_BATCH_SHARED", None)
    assert out["1"][0] == out["0"][0]
    for a, b in zip(out["1"][1], out["0"][1]):
        assert np.array_equal(a, b)

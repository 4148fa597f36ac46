"""Tie rules on the GPU, with weights made to tie exactly:

- the router's rows repeat in triples (rows 3k, 3k+1, 3k+2 equal), so the
  router logits tie in threes at every layer and every top-k boundary splits
  a triple: the selection must keep the lower indices, in ascending order
  inside each tie (the stable rank of qwen35_moe.hex:86-111);
- the vocabulary head's rows repeat with period 97, so every logit value
  occurs at indices m, m + 97, m + 194, ... across the argmax chunks: the
  greedy token must be the first index of the maximum (fused_argmax.hex:
  2-47), always below 97.

Both decode paths against the CPU restatement, whose tie rules are pinned
by closed forms on the CPU (tests/test_oracle_ties.py): tokens, BF16 logits
and every layer's expert ids at every call, bit for bit."""
import numpy as np
import pytest

import cq35
import cq35.config as cc

pytestmark = pytest.mark.gpu

PERIOD = 97


def say(*a):
    print(*a, flush=True)


def tied_weights(oracle, cfg, seed):
    w = oracle.synthetic_weights(cfg, seed)
    specs = oracle.weight_specs(cfg)
    H = cfg["hidden"]
    for i, (_dtype, rows, cols, kind) in enumerate(specs):
        if kind == 6:  # router F32 [E, H]
            r = w[i].reshape(rows, cols)
            for e in range(rows):
                r[e] = r[3 * (e // 3)]
    head = w[len(specs) - 1].reshape(cfg["vocab"], H)
    head[PERIOD:] = np.resize(head[:PERIOD], (cfg["vocab"] - PERIOD, H))
    return w


@pytest.mark.parametrize("name", ["tiny-moe", "mini-moe"])
def test_ties_match_restatement(oracle, name):
    cfg = cc.preset(name)
    w = tied_weights(oracle, cfg, seed=17)
    gm = cq35.Model.from_arrays(cfg, w)
    om = oracle.Model(cfg, w)
    prompt = [5, 900, 17, 3000, 41, 7]
    steps = 12
    cap = len(prompt) + steps + 1
    K = cfg["top_k"]
    for persistent in (True, False):
        say("ties", name, "persistent", persistent)
        os_ = om.session(cap)
        gs = gm.session(cap)
        gs.set_persistent(persistent)
        assert gs.persistent == persistent
        tok_o = tok_g = None
        for pos in range(len(prompt) + steps):
            feed = prompt[pos] if pos < len(prompt) else tok_o
            tok_o, lo = os_.step([feed], pos)
            ids_o = os_.last_ids().reshape(cfg["layers"], K)
            lg, tok_g = gs.step_raw([feed])
            ids_g = gs.router_ids()
            assert np.array_equal(ids_g, ids_o), f"{name}: expert ids differ at position {pos}"
            assert tok_g == tok_o, f"{name}: token {tok_g} vs {tok_o} at position {pos}"
            assert np.array_equal(lg, lo), f"{name}: logits differ at position {pos}"
            # the maximum repeats every PERIOD entries: the first index wins
            f = oracle.bf16_to_f32(lg)
            assert tok_g < PERIOD and f[tok_g] == f.max() and f[tok_g + PERIOD] == f.max()
            # each layer's boundary splits a triple of equal logits: the ids
            # of one triple appear in ascending order, lowest first
            for row in ids_g:
                groups = {}
                for e in row.tolist():
                    groups.setdefault(e // 3, []).append(e)
                for g, members in groups.items():
                    top = min(3, cfg["experts"] - 3 * g)
                    assert members == list(range(3 * g, 3 * g + len(members))), (row, g)
                    assert len(members) == top or g == row[-1] // 3, (row, g)

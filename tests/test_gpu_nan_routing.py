"""Router logits with a NaN, on every selection kernel, against the CPU
restatement.

One router row of every layer is made NaN (expert n = E / 2, never among
the top k: rank(n) = n >= k), so that logit is NaN for every token and the
reference's rank formula (qwen35_moe.hex:86-111),
rank(e) = #{i : l_i > l_e} + #{i < e : !(l_e > l_i)}, counts n among the
lower indices of every expert above it: their ranks move up by one, two
experts can share a rank and a rank can stay unassigned. The restatement
scatters ids[rank] = e in ascending e (the largest index of a shared rank
takes it) and an unassigned rank k keeps expert k; every GPU selection
kernel resolves shared ranks by an LDS maximum to the same result:

- the batched prefill's k_bselect (a multi-token call),
- the persistent step's select_experts and the per-kernel k_router_select
  (one-token calls on both decode paths),
- the weight-shared batched MoE step's k_sselect (cq35_step_batch).

Tokens, BF16 logits and every layer's expert ids at every call, bit for
bit, and the whole state at the end."""
import numpy as np
import pytest

import cq35
import cq35.config as cc

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def nan_weights(oracle, cfg, seed):
    w = oracle.synthetic_weights(cfg, seed)
    specs = oracle.weight_specs(cfg)
    n = cfg["experts"] // 2
    assert n >= cfg["top_k"]
    for i, (_dtype, rows, cols, kind) in enumerate(specs):
        if kind == 6:  # router F32 [E, H]
            w[i].reshape(rows, cols)[n, :] = np.nan
    return w, n


@pytest.mark.parametrize("name", ["tiny-moe", "mini-moe"])
def test_nan_router_logit_matches_restatement(oracle, name):
    cfg = cc.preset(name)
    w, n = nan_weights(oracle, cfg, seed=23)
    gm = cq35.Model.from_arrays(cfg, w)
    om = oracle.Model(cfg, w)
    K, L = cfg["top_k"], cfg["layers"]
    prompt = [5, 900, 17, 3000, 41, 7, 123, 77]
    steps = 10
    cap = len(prompt) + steps + 1
    # restatement: the prompt as one call, then greedy one-token steps
    os_ = om.session(cap)
    tok, lo = os_.step(prompt, 0)
    ref = [(tok, lo, os_.last_ids().reshape(L, K))]
    for i in range(steps):
        tok, lo = os_.step([tok], len(prompt) + i)
        ref.append((tok, lo, os_.last_ids().reshape(L, K)))
    want_state = os_.cache()
    # shared and unassigned ranks occur: an unassigned rank k keeps expert
    # k, which then also holds its own rank in some rows (9 of 44 layer rows
    # on tiny-moe, 11 of 44 on mini-moe)
    repeats = sum(int(len(set(row.tolist())) < K) for _, _, ids in ref for row in ids)
    say(f"  {name}: {repeats} layer rows with a repeated expert")
    assert repeats > 0
    for persistent in (True, False):
        say(name, "persistent", persistent)
        gs = gm.session(cap)
        gs.set_persistent(persistent)
        lg, t = gs.step_raw(prompt)
        got = [(t, lg, gs.router_ids())]
        for _ in range(steps):
            lg, t = gs.step_raw([t])
            got.append((t, lg, gs.router_ids()))
        for c, ((tg, lgg, ig), (tr, lr, ir)) in enumerate(zip(got, ref)):
            assert np.array_equal(ig, ir), f"{name} call {c}: expert ids {ig.tolist()} vs {ir.tolist()}"
            assert tg == tr, f"{name} call {c}: token {tg} vs {tr}"
            assert np.array_equal(lgg, lr), f"{name} call {c}: logits differ"
            assert not (ig == n).any()
        assert np.array_equal(gs.export_state(0), want_state), f"{name}: state differs"


@pytest.mark.parametrize("name", ["tiny-moe", "mini-moe"])
def test_nan_router_logit_batch_matches_alone(oracle, name):
    cfg = cc.preset(name)
    w, _ = nan_weights(oracle, cfg, seed=29)
    gm = cq35.Model.from_arrays(cfg, w)
    B, rounds, cap = 5, 6, 48
    prompts = [[(13 * b + 7 * i) % cfg["vocab"] for i in range(2 + 3 * b)] for b in range(B)]
    group, nxt = [], []
    for p in prompts:
        s = gm.session(cap)
        nxt.append(s.append_next_token(p))
        group.append(s)
    calls = []
    for _ in range(rounds):
        nxt, lg = cq35.decode_batch(group, nxt, logits=True)
        calls.append((list(nxt), lg, [s.router_ids() for s in group]))
    for b in range(B):
        alone = gm.session(cap)
        t = alone.append_next_token(prompts[b])
        for r in range(rounds):
            lg, t2 = alone.step_raw([t])
            assert np.array_equal(calls[r][2][b], alone.router_ids()), f"{name} session {b} round {r}: ids"
            assert calls[r][0][b] == t2 and np.array_equal(calls[r][1][b], lg), f"{name} session {b} round {r}"
            t = t2
        assert np.array_equal(alone.export_state(0), group[b].export_state(0))

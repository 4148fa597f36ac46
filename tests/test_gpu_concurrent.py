"""The long-context serving configuration (8 concurrent sessions at long
context, one chunked matrix-core prefill interleaved between decode rounds):
interleaving changes nothing. Each decode session's greedy tokens and whole
state equal the same session decoded alone, and the interleaved prompt's
state and next token equal the same chunked prompt appended alone, bit for
bit; on the reduced MoE shape above the split-K threshold, and on the
35B-A3B shape at the benchmark's size (8 sessions at 32768 positions, a
4096-token prompt in 1024-token calls on all three matrix-core components)."""
import numpy as np
import pytest
import torch

import cq35
import cq35.config as cc
from test_gpu_long_context import seeded_state

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def run(name, sessions, context, rounds, prompt_len, chunk, components):
    cfg = cc.preset(name)
    m = cq35.Model.synthetic(cfg, seed=21)
    cap = context + rounds + 4
    state = seeded_state(cfg, cap, context, seed=23, device="cuda")
    torch.cuda.empty_cache()
    prompt = np.random.default_rng(5).integers(0, cfg["vocab"], prompt_len).tolist()
    first = [100 + 37 * b for b in range(sessions)]

    def fresh():
        group = []
        for b in range(sessions):
            s = m.session(cap)
            s.import_state(0, state)
            s.position = context
            group.append(s)
        pre = m.session(prompt_len + 4)
        pre.set_matrix_prefill(components)
        return group, pre

    # interleaved: a decode round, then one prefill chunk, until both are done
    group, pre = fresh()
    nxt, hist, done, last = list(first), [], 0, None
    for r in range(rounds):
        nxt = cq35.decode_batch(group, nxt)
        hist.append(list(nxt))
        if done < prompt_len:
            last = pre.append_next_token(prompt[done:done + chunk])
            done += chunk
    while done < prompt_len:
        last = pre.append_next_token(prompt[done:done + chunk])
        done += chunk
    say("  interleaved run done")
    states = [s.export_state(0) for s in group]
    pre_state = pre.export_state(0)
    # alone: each session by itself, then the prompt by itself
    alone, pre2 = fresh()
    for b, s in enumerate(alone):
        t = first[b]
        for r in range(rounds):
            t = s.decode_next_token(t)
            assert t == hist[r][b], f"{name}: session {b} token differs at round {r}"
        assert np.array_equal(s.export_state(0), states[b]), f"{name}: session {b} state differs"
    last2 = None
    for d in range(0, prompt_len, chunk):
        last2 = pre2.append_next_token(prompt[d:d + chunk])
    assert last == last2 and np.array_equal(pre2.export_state(0), pre_state), f"{name}: prefill differs"


ALL3 = cq35.Session.MATRIX_PROJECTIONS | cq35.Session.MATRIX_EXPERTS | cq35.Session.MATRIX_ATTENTION


def test_concurrent_long_context_mini_moe():
    say("concurrent long context, mini-moe")
    run("mini-moe", sessions=8, context=9000, rounds=12, prompt_len=4096, chunk=256,
        components=cq35.Session.MATRIX_PROJECTIONS | cq35.Session.MATRIX_EXPERTS)


@pytest.mark.timeout(600)
def test_concurrent_long_context_35b_full_size():
    """The benchmark's configuration 5 as measured: 8 sessions at 32768
    cached positions, a 4096-token prompt appended in 1024-token calls (the
    reference server's prefill block) with all three matrix-core components,
    interleaved with the decode rounds."""
    say("concurrent long context, qwen36-35b-a3b, full size")
    run("qwen36-35b-a3b", sessions=8, context=32768, rounds=8, prompt_len=4096, chunk=1024, components=ALL3)

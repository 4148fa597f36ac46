"""cq35_step_batch: one decode step for several independent sessions gives
every session exactly what stepping it alone gives (tokens and the whole
state, bit for bit), for per-kernel sessions (overlapped launches), persistent
sessions and a mix of both models; the batch checks every entry before any
work."""
import numpy as np
import pytest

import cq35
import cq35.config as cc

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def prompts(cfg, count):
    rng = np.random.default_rng(count)
    return [rng.integers(0, cfg["vocab"], 3 + 2 * i).tolist() for i in range(count)]


def test_batch_matches_sessions_stepped_alone():
    dense = cq35.Model.synthetic(cc.preset("mini"), seed=7)
    moe = cq35.Model.synthetic(cc.preset("mini-moe"), seed=8)
    say("batch of dense + MoE sessions")
    plan = [(dense, p) for p in prompts(dense.cfg, 4)] + [(moe, p) for p in prompts(moe.cfg, 3)]
    batch, alone, nxt_b, nxt_a = [], [], [], []
    for i, (m, p) in enumerate(plan):
        for group, nxt in ((batch, nxt_b), (alone, nxt_a)):
            s = m.session(64)
            if i < 2:
                s.set_persistent(False)  # two dense sessions on the per-kernel path
            nxt.append(s.append_next_token(p))
            group.append(s)
    assert nxt_b == nxt_a
    assert any(s.persistent for s in batch) and not all(s.persistent for s in batch)
    for step in range(10):
        nxt_b = cq35.decode_batch(batch, nxt_b)
        nxt_a = [s.decode_next_token(t) for s, t in zip(alone, nxt_a)]
        assert nxt_b == nxt_a, f"step {step}"
    for sb, sa in zip(batch, alone):
        assert sb.position == sa.position
        assert np.array_equal(sb.export_state(0), sa.export_state(0))


def test_batch_rejects_before_any_work():
    m = cq35.Model.synthetic(cc.preset("mini"), seed=7)
    a, b = m.session(8), m.session(8)
    a.append_next_token([1, 2])
    b.append_next_token([3, 4, 5, 6, 7, 8, 9])
    state = a.export_state(0)
    from cq35 import _lib
    import ctypes
    lib = _lib.load()
    h = (ctypes.c_void_p * 2)(a._h.value, a._h.value)
    toks = np.array([1, 1], dtype=np.uint64)
    starts = np.array([2, 2], dtype=np.int64)
    out = np.zeros(2, dtype=np.uint64)
    assert lib.cq35_step_batch(h, toks.ctypes.data, starts.ctypes.data, 2, out.ctypes.data, None) == -1  # twice
    h = (ctypes.c_void_p * 2)(a._h.value, b._h.value)
    starts = np.array([2, 8], dtype=np.int64)
    assert lib.cq35_step_batch(h, toks.ctypes.data, starts.ctypes.data, 2, out.ctypes.data, None) == -2  # capacity
    toks = np.array([1, m.cfg["vocab"]], dtype=np.uint64)
    starts = np.array([2, 7], dtype=np.int64)
    assert lib.cq35_step_batch(h, toks.ctypes.data, starts.ctypes.data, 2, out.ctypes.data, None) == -2  # vocabulary
    assert np.array_equal(a.export_state(0), state), "a rejected batch must not touch any session"

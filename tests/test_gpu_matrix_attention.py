"""Matrix-core attention of the prompt path (CQ35_MATRIX_ATTENTION, the
reference's matrix-core attention component, qwen35_wmma_attention.hex).

- The kernel alone, through cq35_device_matrix_attention, against a float64
  statement with the reference's rounding points: score bf16(q.k * scale)
  with keys after the row's position masked, probability
  bf16(exp(s - max) / den), output bf16(bf16(sum p v) * sigmoid(gate)). The
  products' F32 sums run in the hardware's order, so the bar is a tolerance;
  a CPU test shows that plausible mistakes (a causal mask off by one, the
  scale missing, probabilities left unnormalised, the wrong KV head, the gate
  dropped) land far outside it.
- Whole prompts with the component on: within the reference's 5% gate of the
  exact staged attention, also for a second call that continues a cached
  context (rows at positions past the chunk start)."""
import numpy as np
import pytest

import cq35
import cq35.config as cc
from cq35.model import Session

ATT = Session.MATRIX_ATTENTION
ALL3 = Session.MATRIX_PROJECTIONS | Session.MATRIX_EXPERTS | Session.MATRIX_ATTENTION


def say(*a):
    print(*a, flush=True)


def to_bf(a):  # round to nearest even
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf2f(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def rbf(x):
    return bf2f(to_bf(np.asarray(x, dtype=np.float32))).astype(np.float64)


def rel_rms(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.sqrt(np.mean((a - b) ** 2)) / np.sqrt(np.mean(b ** 2)))


def statement(q, gate, k, v, start, heads, kv_heads, hd, plant=None):
    """float64 attention with the reference's BF16 rounding points."""
    n = q.shape[0]
    keys = start + n
    qf = bf2f(q).reshape(n, heads, hd).astype(np.float64)
    gf = bf2f(gate).reshape(n, heads, hd).astype(np.float64)
    kf = bf2f(k).reshape(keys, kv_heads, hd).astype(np.float64)
    vf = bf2f(v).reshape(keys, kv_heads, hd).astype(np.float64)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    if plant == "no scale":
        scale = np.float32(1.0)
    pos = start + np.arange(n)
    mask = np.arange(keys)[None, :] > pos[:, None]
    if plant == "mask off by one":
        mask = np.arange(keys)[None, :] >= pos[:, None]
        mask[:, 0] = False
    out = np.empty((n, heads, hd))
    group = heads // kv_heads
    for h in range(heads):
        kv = h // group
        if plant == "wrong kv head":
            kv = (kv + 1) % kv_heads
        s = rbf((qf[:, h, :] @ kf[:, kv, :].T).astype(np.float32) * scale)
        s[mask] = -np.inf
        m = s.max(axis=1, keepdims=True)
        e = np.exp(s - m)
        e[mask] = 0.0
        p = e if plant == "unnormalised" else rbf(e / e.sum(axis=1, keepdims=True))
        ctx = rbf(p @ vf[:, kv, :])
        g = 1.0 if plant == "no gate" else 1.0 / (1.0 + np.exp(-gf[:, h, :]))
        out[:, h, :] = rbf(ctx * g)
    return out.reshape(n, heads * hd)


def case(seed, n, start, heads, kv_heads, hd, qscale=3.0):
    rng = np.random.default_rng(seed)
    keys = start + n
    q = to_bf(rng.standard_normal((n, heads * hd)) * qscale)
    gate = to_bf(rng.standard_normal((n, heads * hd)))
    k = to_bf(rng.standard_normal((keys, kv_heads * hd)))
    v = to_bf(rng.standard_normal((keys, kv_heads * hd)))
    return q, gate, k, v


# the bar: relative RMS against the float64 statement, and the share of
# outputs more than 4 BF16 units in the last place away
REL_RMS = 1e-2
FAR_SHARE = 2e-3


def far_share(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    ulp = np.maximum(np.abs(b), 1e-3) * 2.0 ** -8
    return float(np.mean(np.abs(a - b) > 4 * ulp))


SHAPES = [  # n, start, heads, kv_heads, head_dim
    (1, 0, 4, 2, 64),
    (37, 0, 4, 2, 64),
    (100, 300, 16, 2, 256),
    (64, 1000, 8, 2, 128),
    (33, 4000, 16, 2, 256),
    (300, 0, 8, 1, 256),
]


def test_tolerance_rejects_planted_mistakes():
    """CPU: every planted mistake in the statement misses one of the two bars
    by more than five times."""
    for n, start, heads, kvh, hd in [(37, 0, 4, 2, 64), (40, 200, 8, 2, 256)]:
        q, gate, k, v = case(1, n, start, heads, kvh, hd)
        good = statement(q, gate, k, v, start, heads, kvh, hd)
        for plant in ["mask off by one", "no scale", "unnormalised", "wrong kv head", "no gate"]:
            bad = statement(q, gate, k, v, start, heads, kvh, hd, plant)
            r, f = rel_rms(bad, good), far_share(bad, good)
            assert max(r / REL_RMS, f / FAR_SHARE) > 5, (plant, r, f)


def device_attention(q, gate, k, v, n, start, heads, kv_heads, hd):
    from cq35 import _lib
    out = np.empty((n, heads * hd), dtype=np.uint16)
    rc = _lib.load().cq35_device_matrix_attention(q.ctypes.data, gate.ctypes.data, k.ctypes.data, v.ctypes.data,
                                                  n, start, heads, kv_heads, hd, out.ctypes.data)
    assert rc == 0, _lib.load().cq35_last_error()
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("n,start,heads,kv_heads,hd", SHAPES)
def test_matrix_attention_against_f64(n, start, heads, kv_heads, hd):
    say("matrix attention: rows", n, "start", start, "heads", heads, "kv heads", kv_heads, "head dim", hd)
    q, gate, k, v = case(n + start, n, start, heads, kv_heads, hd)
    got = bf2f(device_attention(q, gate, k, v, n, start, heads, kv_heads, hd))
    want = statement(q, gate, k, v, start, heads, kv_heads, hd)
    assert np.all(np.isfinite(got))
    r, f = rel_rms(got, want), far_share(got, want)
    say(f"  relative RMS {r:.2e}, share beyond 4 ulp {f:.2e}")
    assert r <= REL_RMS and f <= FAR_SHARE


def test_matrix_attention_rejects_bad_shapes():
    """CPU: shapes the kernel does not take fail before any device work."""
    from cq35 import _lib
    lib = _lib.load()
    q = np.zeros(4 * 256, dtype=np.uint16)
    p = q.ctypes.data
    for n, start, heads, kvh, hd in [(1, 0, 4, 2, 96), (0, 0, 4, 2, 64), (1, -1, 4, 2, 64), (1, 0, 4, 3, 64),
                                     (1, 0, 0, 1, 64), (1, 1 << 20, 4, 2, 64)]:
        assert lib.cq35_device_matrix_attention(p, p, p, p, n, start, heads, kvh, hd, p) != 0
        assert b"bad matrix attention shape" in lib.cq35_last_error()


def logits_f32(bits):
    return bf2f(bits)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["mini", "mini-moe", "tiny"])
@pytest.mark.parametrize("components", [ATT, ALL3])
def test_matrix_attention_prompts_within_reference_gate(name, components):
    cfg = dict(cc.preset(name))
    if not cfg["moe"]:
        components &= ~Session.MATRIX_EXPERTS
    say("matrix attention prompts", name, "components", components)
    m = cq35.Model.synthetic(cfg, seed=5)
    rng = np.random.default_rng(3)
    first = rng.integers(0, cfg["vocab"], 300).tolist()
    second = rng.integers(0, cfg["vocab"], 77).tolist()
    se, sm = m.session(400), m.session(400)
    sm.set_matrix_prefill(components)
    for i, prompt in enumerate([first, second]):
        le, te = se.step_raw(prompt)
        lm, tm = sm.step_raw(prompt)
        r = rel_rms(logits_f32(lm), logits_f32(le))
        say(f"  call {i} ({len(prompt)} rows): relative logit RMS {r:.4f}, tokens {te} / {tm}")
        assert np.all(np.isfinite(logits_f32(lm)))
        assert r <= 0.05, f"call {i}: relative logit RMS {r:.4f} above the 5% gate"
    r = rel_rms(logits_f32(sm.export_state(0)), logits_f32(se.export_state(0)))
    say(f"  session state relative RMS {r:.4f}")
    assert r <= 0.05

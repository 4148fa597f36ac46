"""Per-function pins of the CPU restatement (oracle/) against independent
float64 formulations, on BF16-representable inputs.

Each restated function is compared with the textbook mathematics of the
operation (the reference's rounding points are not restated in the float64
side); the tolerance is a relative RMS error derived from the number of
BF16 roundings on the function's path, with U = 2^-8 the BF16 unit roundoff
(8 significant bits; one rounding has a relative RMS error of about
U / sqrt(3)). For every plausible mistake the restatement is then run with
that mistake planted (oracle.planted) and must miss the float64 result by at
least 3x the tolerance, on every shape where the mistake changes the
mathematics. Shapes: `tiny` (head_dim 64, rotary 16, key/value dim 32) and
`mini-moe` (head_dim 256, rotary 64, key/value dim 128: the 35B-A3B head
shapes)."""
import ctypes

import numpy as np
import pytest

import cq35.config as cc

U = 2.0 ** -8
SHAPES = ["tiny", "mini-moe"]
MARGIN = 3.0


def bf16(oracle, a):
    return oracle.bf16_round(np.asarray(a, dtype=np.float32))


def f64(oracle, bits):
    return oracle.bf16_to_f32(bits).astype(np.float64)


def rel_rms(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return float(np.sqrt(np.mean((got - ref) ** 2)) / np.sqrt(np.mean(ref ** 2)))


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


_models = {}


def model(oracle, name):
    """A restatement model of the shape (its weights are not used here)."""
    if name not in _models:
        cfg = cc.preset(name)
        w = oracle.synthetic_weights(cfg, 1)
        _models[name] = (cfg, oracle.Model(cfg, w))
    return _models[name]


def check(oracle, measure, tol, plants, label):
    """measure() -> relative RMS error of the restatement; within tol, and
    each planted mistake at least MARGIN x tol."""
    base = measure()
    assert base <= tol, f"{label}: restatement off by {base:.3g} > {tol:.3g}"
    for p in plants:
        with oracle.planted(p):
            bad = measure()
        assert bad >= MARGIN * tol, f"{label}: planted {p} only {bad:.3g} < {MARGIN} x {tol:.3g}"
    return base


# ------------------------------------------------------------------ RoPE

def rope_f64(oracle, cfg, x, position):
    """neox rotation of the first R channels by position * theta^(-2i/R); the
    frequencies are the reference's F32 constants (host powf,
    src/catena.rs:185-232) and the angle their F32 product with the position;
    cos/sin and the rotation in float64."""
    R, HD = cfg["rope_dim"], cfg["head_dim"]
    half = R // 2
    i = np.arange(half, dtype=np.float32)
    freq = np.power(np.float32(cfg["theta"]), -(np.float32(2.0) * i / np.float32(R))).astype(np.float32)
    ang = (np.float32(np.uint32(position)) * freq).astype(np.float32).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    y = x.copy()
    a, b = x[..., :half], x[..., half:R]
    y[..., :half] = a * c - b * s
    y[..., half:R] = b * c + a * s
    return y


@pytest.mark.parametrize("name", SHAPES)
@pytest.mark.parametrize("position", [3, 1000, 65537, 131071])
def test_rope_pinned(oracle, name, position):
    cfg, m = model(oracle, name)
    heads, HD = 6, cfg["head_dim"]
    x = bf16(oracle, np.random.default_rng(position).standard_normal((heads, HD)))
    out = np.empty_like(x)

    def measure():
        oracle.lib().ox_k_rope(m._h, position, ptr(x), heads, ptr(out))
        return rel_rms(f64(oracle, out), rope_f64(oracle, cfg, f64(oracle, x), position))

    # one BF16 rounding of the output (the F32 products and sincos add ~2^-22)
    check(oracle, measure, U, ["rope_pairing", "rope_sign", "rope_freq_hd"], f"rope {name} @{position}")


@pytest.mark.parametrize("name", SHAPES)
def test_head_norm_and_rope_pinned(oracle, name):
    """full_prepare: head RMS (adjacent-pair tree) with the norm weights,
    then RoPE. Weights spread 1 +- 0.5 so a dropped weight shows."""
    cfg, m = model(oracle, name)
    heads, HD = 5, cfg["head_dim"]
    rng = np.random.default_rng(7)
    x = bf16(oracle, rng.standard_normal((heads, HD)) * 3.0)
    w = (1.0 + rng.uniform(-0.5, 0.5, HD)).astype(np.float32)
    out = np.empty_like(x)
    position = 777

    def measure():
        oracle.lib().ox_k_prepare_heads(m._h, position, ptr(x), ptr(w), heads, ptr(out))
        xf = f64(oracle, x)
        n = xf / np.sqrt(np.mean(xf * xf, axis=1, keepdims=True) + cfg["eps"]) * w.astype(np.float64)
        return rel_rms(f64(oracle, out), rope_f64(oracle, cfg, n, position))

    # bf16(x * inv), bf16(w), their BF16 product, the rotated output: 4 roundings
    check(oracle, measure, 2 * U, ["norm_weight", "rope_sign", "rope_pairing"], f"head norm {name}")


def test_hidden_norm_pinned(oracle):
    rng = np.random.default_rng(3)
    for cols in (256, 1000, 2048):
        x = bf16(oracle, rng.standard_normal((3, cols)) * 5.0)
        w = (1.0 + rng.uniform(-0.5, 0.5, cols)).astype(np.float32)
        out = np.empty_like(x)

        def measure():
            oracle.lib().ox_k_normalize(ptr(x), ptr(w), cols, 3, ctypes.c_float(1e-6), ptr(out))
            xf = f64(oracle, x)
            ref = xf / np.sqrt(np.mean(xf * xf, axis=1, keepdims=True) + 1e-6) * w
            return rel_rms(f64(oracle, out), ref)

        # bf16(x * inv), bf16(w), the BF16 product: 3 roundings
        check(oracle, measure, 2 * U, ["norm_weight"], f"hidden norm {cols}")


# ------------------------------------------------------------ DeltaNet

@pytest.mark.parametrize("name", SHAPES)
@pytest.mark.parametrize("position", [1, 2, 9])
def test_conv_pinned(oracle, name, position):
    """4-tap causal conv over (history slots of positions p-3, p-2, p-1, the
    current row) with zero taps before position 0, then SiLU; the current
    row replaces history slot p mod 3."""
    cfg, m = model(oracle, name)
    d = cc.derived(cfg)
    QKV = d["qkv"]
    rng = np.random.default_rng(position)
    hist = bf16(oracle, rng.standard_normal((3, QKV)))
    qkv = bf16(oracle, rng.standard_normal(QKV))
    w = (rng.standard_normal((QKV, 4)) * 0.3).astype(np.float32)
    out = np.empty(QKV, dtype=np.uint16)
    work = hist.copy()

    def measure():
        work[:] = hist
        oracle.lib().ox_k_conv(m._h, ptr(work), position, ptr(w), ptr(qkv), ptr(out))
        window = np.zeros((4, QKV))
        for t in range(3):  # tap t reads position p - 3 + t, held in slot (p + t) mod 3
            if position - 3 + t >= 0:
                window[t] = f64(oracle, hist[(position + t) % 3])
        window[3] = f64(oracle, qkv)
        s = np.sum(window.T * w.astype(np.float64), axis=1)
        ref = s / (1.0 + np.exp(-s))
        return rel_rms(f64(oracle, out), ref)

    # BF16 of the sum, then of the SiLU output (SiLU's slope stays below 1.1)
    check(oracle, measure, 2 * U, ["conv_tap_order"] if position >= 2 else [], f"conv {name} @{position}")
    expect = hist.copy()
    expect[position % 3] = qkv
    assert np.array_equal(work, expect), "history slot update"


@pytest.mark.parametrize("name", SHAPES)
def test_l2_pinned(oracle, name):
    cfg, _ = model(oracle, name)
    KH, KD = cfg["key_heads"], cfg["key_dim"]
    x = bf16(oracle, np.random.default_rng(5).standard_normal((KH, KD)) * np.arange(1, KH + 1)[:, None])
    out = np.empty_like(x)

    def measure():
        oracle.lib().ox_k_l2(ptr(x), KH, KD, ptr(out))
        xf = f64(oracle, x)
        return rel_rms(f64(oracle, out), xf / np.sqrt(np.sum(xf * xf, axis=1, keepdims=True) + 1e-6))

    check(oracle, measure, U, ["l2_whole"], f"l2 {name}")


def delta_f64(cfg, v, q, k, alpha, beta, dt, a, S, key_head):
    """Gated delta rule for every value head h (key head key_head(h)):
    g = exp(softplus(alpha + dt) * a), b = sigmoid(beta);
    S' = g S + (b (v - g S k)) k^T;  o = S' q / sqrt(KD)."""
    VH, VD, KD = cfg["value_heads"], cfg["value_dim"], cfg["key_dim"]
    S2 = np.empty_like(S)
    o = np.empty((VH, VD))
    for h in range(VH):
        j = key_head(h)
        x = alpha[h] + dt[h]
        g = np.exp((np.maximum(x, 0) + np.log1p(np.exp(-abs(x)))) * a[h])
        b = 1.0 / (1.0 + np.exp(-beta[h]))
        delta = (v[h] - g * (S[h] @ k[j])) * b
        S2[h] = g * S[h] + np.outer(delta, k[j])
        o[h] = S2[h] @ q[j] / np.sqrt(KD)
    return S2, o


@pytest.mark.parametrize("name", SHAPES)
def test_delta_pinned(oracle, name):
    """cached_delta / register_delta: state BF16 in the cache (decode) or
    F32 in the shadow (multi-token calls)."""
    cfg, m = model(oracle, name)
    d = cc.derived(cfg)
    KH, KD, VH, VD = cfg["key_heads"], cfg["key_dim"], cfg["value_heads"], cfg["value_dim"]
    KS, VS = d["key_size"], d["value_size"]
    rng = np.random.default_rng(13)
    # unit-norm q, k (as after the L2 norms), BF16
    def unit(n):
        x = rng.standard_normal((n, KD))
        return bf16(oracle, x / np.linalg.norm(x, axis=1, keepdims=True))
    q, k = unit(KH), unit(KH)
    conv = np.zeros(d["qkv"], dtype=np.uint16)
    conv[2 * KS:] = bf16(oracle, rng.standard_normal(VS))
    alpha = bf16(oracle, rng.standard_normal(VH))
    beta = bf16(oracle, rng.standard_normal(VH))
    dt = np.ones(VH, dtype=np.float32)
    a = (-(1.0 + 15.0 * rng.uniform(0, 1, VH))).astype(np.float32)
    S0 = bf16(oracle, rng.standard_normal((VH, VD, KD)))
    r = VH // KH
    for f32_state in (False, True):
        state16 = S0.copy()
        state32 = f64(oracle, S0).astype(np.float32)
        out = np.empty(VS, dtype=np.uint16)

        def measure():
            state16[:] = S0
            state32[:] = f64(oracle, S0)
            oracle.lib().ox_k_delta(m._h, ptr(conv), ptr(q), ptr(k), ptr(alpha), ptr(beta), ptr(dt), ptr(a),
                                    None if f32_state else ptr(state16), ptr(state32) if f32_state else None,
                                    ptr(out))
            S2, o = delta_f64(cfg, f64(oracle, conv[2 * KS:]).reshape(VH, VD), f64(oracle, q), f64(oracle, k),
                              f64(oracle, alpha), f64(oracle, beta), dt.astype(np.float64),
                              a.astype(np.float64), f64(oracle, S0), lambda h: h % KH)
            got_S = state32.astype(np.float64) if f32_state else f64(oracle, state16)
            return max(rel_rms(f64(oracle, out).reshape(VH, VD), o), rel_rms(got_S, S2))

        # roundings: the gate's softplus * a to BF16 (an absolute error of
        # U |softplus * a| in the exponent, so relative U |softplus * a| in
        # the decay, which weighs little where |softplus * a| is large),
        # sigmoid(beta) to BF16, the stored state (BF16 decode), the output:
        # 2U (measured 0.6-0.9U)
        plants = ["delta_scale", "delta_pred_decay"] + (["key_head"] if r > 1 else [])
        check(oracle, measure, 2 * U, plants, f"delta {name} f32={f32_state}")


@pytest.mark.parametrize("name", SHAPES)
def test_gated_norm_pinned(oracle, name):
    cfg, m = model(oracle, name)
    VH, VD = cfg["value_heads"], cfg["value_dim"]
    rng = np.random.default_rng(17)
    core = bf16(oracle, rng.standard_normal((VH, VD)) * 0.3)
    z = bf16(oracle, rng.standard_normal((VH, VD)))
    w = (1.0 + rng.uniform(-0.5, 0.5, VD)).astype(np.float32)
    out = np.empty_like(core)

    def measure():
        oracle.lib().ox_k_gated_norm(m._h, ptr(core), ptr(z), ptr(w), ptr(out))
        c, zf = f64(oracle, core), f64(oracle, z)
        ref = c / np.sqrt(np.mean(c * c, axis=1, keepdims=True) + cfg["eps"]) * w * (zf / (1 + np.exp(-zf)))
        return rel_rms(f64(oracle, out), ref)

    # one BF16 rounding of the output; F32 division, SiLU and products add ~2^-21
    check(oracle, measure, U, ["gated_sum"], f"gated norm {name}")


# ------------------------------------------------------------ attention

def attention_f64(cfg, q, K, V, gate):
    Q, KVH, HD = cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"]
    out = np.empty((Q, HD))
    for h in range(Q):
        g = h // (Q // KVH)
        s = K[:, g] @ q[h] / np.sqrt(HD)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = (p @ V[:, g]) / (1.0 + np.exp(-gate[h]))
    return out


@pytest.mark.parametrize("name", ["tiny-moe", "mini-moe", "tiny"])
@pytest.mark.parametrize("keys,split", [(1, 0), (13, 0), (4100, 0), (13, 8), (4100, 1000)])
def test_attention_pinned(oracle, name, keys, split):
    """Online 8-key-tile softmax (MoE decode) and the dense staged attention,
    over `keys` cached rows like the long-context state (K rows of a unit
    head RMS, V ~ 0.1 N(0,1))."""
    cfg, m = model(oracle, name)
    Q, KVH, HD = cfg["q_heads"], cfg["kv_heads"], cfg["head_dim"]
    rng = np.random.default_rng(keys)
    q = bf16(oracle, rng.standard_normal((Q, HD)))
    K = bf16(oracle, rng.standard_normal((keys, KVH, HD)))
    V = bf16(oracle, rng.standard_normal((keys, KVH, HD)) * 0.1)
    qg = bf16(oracle, rng.standard_normal((Q, 2, HD)))  # [q | gate] per head; gate half used
    kv = np.concatenate([K.reshape(-1), V.reshape(-1)])
    out = np.empty((Q, HD), dtype=np.uint16)
    online = 1 if cfg["moe"] else 0

    def measure():
        oracle.lib().ox_k_attention(m._h, online, ptr(q), ptr(kv), keys, ptr(qg), split, ptr(out))
        ref = attention_f64(cfg, f64(oracle, q), f64(oracle, K), f64(oracle, V), f64(oracle, qg[:, 1]))
        return rel_rms(f64(oracle, out), ref)

    plants = ["attn_scale"] if keys > 1 else []
    if Q // KVH > 1 and KVH > 1 and keys > 1:
        plants.append("gqa_map")
    # online: bf16(acc / den), then the gated BF16 output: 2 roundings.
    # staged: scores rounded to BF16 before the softmax (relative error of p
    # up to U |s|, |s| <~ 4 here, averaging out over the keys), p in BF16,
    # the context in BF16, the gated output: 4U (measured 0.5-1.2U)
    tol = 2 * U if online else 4 * U
    check(oracle, measure, tol, plants, f"attention {name} keys={keys} split={split}")


# ------------------------------------------------- whole decode steps

def spread_qk_norms(cfg, weights, rng):
    """q_norm / k_norm weights 1 + U(-0.5, 0.5), so a swapped pair changes
    the attention by far more than BF16 noise."""
    from textbook import Textbook
    tb = Textbook(cfg, weights)
    for l in range(cfg["layers"]):
        if tb.full[l]:
            for slot in (5, 6):
                w = weights[tb.base[l] + slot]
                w[:] = (1.0 + rng.uniform(-0.5, 0.5, w.size)).astype(np.float32)


def state_views(cfg, cache, capacity, position):
    """(K rows, V rows) of every full layer for positions < position, and
    every linear layer's DeltaNet state, from a BF16 cache."""
    d = cc.derived(cfg)
    L, KVS = cfg["layers"], d["kvs"]
    kv = cache[:L * 2 * capacity * KVS].reshape(L, 2, capacity, KVS)
    tail = cache[L * 2 * capacity * KVS:].reshape(L, -1)
    full = [l for l in range(L) if cc.is_full(cfg, l)]
    lin = [l for l in range(L) if not cc.is_full(cfg, l)]
    return ([kv[l, 0, :position] for l in full], [kv[l, 1, :position] for l in full],
            [tail[l, d["conv"]:] for l in lin])


def textbook_views(cfg, tb):
    full = [l for l in range(cfg["layers"]) if tb.full[l]]
    lin = [l for l in range(cfg["layers"]) if not tb.full[l]]
    return ([np.stack(tb.K[l]).reshape(len(tb.K[l]), -1) for l in full],
            [np.stack(tb.V[l]).reshape(len(tb.V[l]), -1) for l in full],
            [tb.S[l].reshape(-1) for l in lin])


def state_error(oracle, cfg, cache, capacity, position, tb):
    ok, ov, os_ = state_views(cfg, cache, capacity, position)
    tk, tv, ts = textbook_views(cfg, tb)
    err = 0.0
    for a, b in zip(ok + ov + os_, tk + tv + ts):
        err = max(err, rel_rms(f64(oracle, a).reshape(b.shape), b))
    return err


@pytest.mark.parametrize("name", ["tiny", "tiny-moe", "mini-moe"])
def test_decode_state_pinned(oracle, name):
    """Six prompt tokens and three greedy steps, one token per call: every
    cached K and V row of the full-attention layers and every DeltaNet state
    against the float64 textbook (fed the restatement's tokens). Within BF16
    activation noise; planted mistakes in the head norms, RoPE, conv taps,
    the delta rule and (MoE) the expert routing miss by far more."""
    from textbook import Textbook
    cfg = cc.preset(name)
    rng = np.random.default_rng(31)
    weights = oracle.synthetic_weights(cfg, 5)
    spread_qk_norms(cfg, weights, rng)
    tokens = rng.integers(0, cfg["vocab"], 6).tolist()
    steps = 3
    cap = len(tokens) + steps + 1

    def measure():
        m = oracle.Model(cfg, weights)
        s = m.session(cap)
        tb = Textbook(cfg, weights)
        feed = list(tokens)
        for pos in range(len(tokens) + steps):
            nxt, _ = s.step([feed[pos]], pos)
            tb.step(feed[pos], pos)
            if pos + 1 >= len(tokens):
                feed.append(nxt)
        return state_error(oracle, cfg, s.cache(), cap, len(tokens) + steps, tb)

    # BF16 activations through up to 4 layers (two or three roundings per
    # layer on the residual path, relative, plus the norms' re-scaling):
    # 12U (measured 0.029-0.037, i.e. 7.4-9.5U)
    plants = ["qk_norm_swap", "rope_sign", "rope_pairing", "rope_freq_hd", "conv_tap_order",
              "delta_pred_decay", "delta_scale", "norm_weight"]
    if cfg["value_heads"] > cfg["key_heads"]:
        plants.append("key_head")
    if cfg["moe"]:
        # routing semantics (moe.hex:86-252, 254-369): descending selection,
        # weights renormalised over the top k only, the shared expert's
        # sigmoid gate
        plants += ["select_ascending", "prob_unnormalised", "softmax_all", "shared_gate"]
    check(oracle, measure, 12 * U, plants, f"decode state {name}")


@pytest.mark.parametrize("name", ["tiny", "mini-moe"])
def test_long_position_step_pinned(oracle, name):
    """One decode step at position 5000 from an imported seeded state (K/V
    rows, conv history and DeltaNet state ~ the long-context configuration's):
    the logits, the new K/V rows and the updated state against the textbook
    run from the same state. RoPE at large angles and attention over 5000
    keys are on this path."""
    from textbook import Textbook
    cfg = cc.preset(name)
    rng = np.random.default_rng(41)
    weights = oracle.synthetic_weights(cfg, 6)
    spread_qk_norms(cfg, weights, rng)
    position, cap = 5000, 5002
    m0 = oracle.Model(cfg, weights)
    n = len(m0.session(cap).cache())
    d = cc.derived(cfg)
    L, KVS = cfg["layers"], d["kvs"]
    state = np.zeros(n, dtype=np.uint16)
    kv = state[:L * 2 * cap * KVS].reshape(L, 2, cap, KVS)
    kv[:, :, :position] = bf16(oracle, rng.standard_normal((L, 2, position, KVS)) * 0.1)
    # keys as stored by the prepare step: unit head RMS, rotated
    kv[:, 0, :position] = bf16(oracle, rng.standard_normal((L, position, KVS)))
    tail = state[L * 2 * cap * KVS:].reshape(L, -1)
    tail[:, :d["conv"]] = bf16(oracle, rng.standard_normal((L, d["conv"])) * 0.1)
    tail[:, d["conv"]:] = bf16(oracle, rng.standard_normal((L, tail.shape[1] - d["conv"])))
    token = 77

    def measure():
        m = oracle.Model(cfg, weights)
        s = m.session(cap)
        s.import_cache(state)
        _, logits = s.step([token], position)
        tb = Textbook(cfg, weights)
        tb.import_cache(state, cap, position)
        ref = tb.step(token, position)
        ok, ov, os_ = state_views(cfg, s.cache(), cap, position + 1)
        tk, tv, ts = textbook_views(cfg, tb)
        # the step's own K / V rows (the imported ones are equal on both sides)
        new_rows = [rel_rms(f64(oracle, a[-1]), b[-1]) for a, b in zip(ok + ov, tk + tv)]
        states = [rel_rms(f64(oracle, a), b) for a, b in zip(os_, ts)]
        return max([rel_rms(f64(oracle, logits), ref)] + new_rows + states)

    # one step through every layer from BF16 state: 10U (measured 0.018-0.024)
    check(oracle, measure, 10 * U, ["qk_norm_swap", "rope_sign", "rope_pairing", "rope_freq_hd", "attn_scale",
                                  "conv_tap_order", "delta_pred_decay"], f"long position {name}")

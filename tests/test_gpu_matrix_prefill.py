"""Matrix-core prefill (MFMA, hardware accumulation order) against the exact
SIMT prefill, which the other GPU tests pin bit for bit to the CPU
restatement.

- The MFMA product itself: against F64 products of the same BF16 operands,
  within BF16 output rounding plus the F32 accumulation bound.
- Whole prompts on shallow shapes (4 layers): the reference's accuracy gate
  for its own matrix-core prefill (PREFILL_BENCHMARKS.md:83, 105), at most 5%
  relative logit RMS, for the logits and for the session state, with decoding
  continued from it.
- The 40-layer 35B-A3B shape with random-init weights amplifies any change
  of accumulation order layer by layer: the reference's own two exact orders
  (batched B256 prefill and token-by-token S256 decode) differ there by
  about as much. The bar is that the matrix-core prompt stays within that
  spread of the exact batched one.
- The switch leaves decode steps and the exact path untouched."""
import numpy as np
import pytest

import cq35
import cq35.config as cc
from cq35.model import Session

pytestmark = pytest.mark.gpu

ALL = Session.MATRIX_PROJECTIONS | Session.MATRIX_EXPERTS


def say(*a):
    print(*a, flush=True)


def logits_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def rel_rms(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.sqrt(np.mean((a - b) ** 2)) / np.sqrt(np.mean(b ** 2)))


def prefill(model, prompt, components, capacity, decode=0):
    s = model.session(capacity)
    s.set_matrix_prefill(components)
    assert s.matrix_prefill == components
    logits, tok = s.step_raw(prompt)
    out = [(tok, logits)]
    for _ in range(decode):
        logits, tok = s.step_raw([tok])
        out.append((tok, logits))
    return s, out


def shape(name):
    """A preset, or 'preset@L' for the same dimensions with L layers."""
    base, _, layers = name.partition("@")
    cfg = dict(cc.preset(base))
    if layers:
        cfg["layers"] = int(layers)
    return cfg


def to_bf(a):  # round to nearest even
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def device_gemm(x, w, w2, res, n, rows, cols, mode, kernel):
    from cq35 import _lib
    out = np.empty((n, rows), dtype=np.uint16)
    ptr = lambda a: a.ctypes.data if a is not None else None
    rc = _lib.load().cq35_device_matrix_gemm(ptr(x), ptr(w), ptr(w2), ptr(res), n, rows, cols, mode, kernel,
                                             out.ctypes.data)
    assert rc == 0
    return out


@pytest.mark.parametrize("kernel", [0, 1])
@pytest.mark.parametrize("n,rows,cols", [(1, 1, 16), (37, 70, 48), (300, 130, 2048),
                                         (96, 32, 4096), (256, 1100, 512)])
def test_matrix_gemm_against_f64(n, rows, cols, kernel):
    say("matrix gemm", n, rows, cols, "kernel", kernel)
    rng = np.random.default_rng(rows + cols)
    x = to_bf(rng.standard_normal((n, cols)))
    w = to_bf(rng.standard_normal((rows, cols)) * 0.05)
    out = device_gemm(x, w, None, None, n, rows, cols, 0, kernel)
    xf = logits_f32(x).astype(np.float64).reshape(n, cols)
    wf = logits_f32(w).astype(np.float64).reshape(rows, cols)
    ref = xf @ wf.T
    mag = np.abs(xf) @ np.abs(wf).T
    y = logits_f32(out).astype(np.float64).reshape(n, rows)
    bound = 2.0 ** -8 * np.abs(ref) + (1 + 2.0 ** -8) * cols * 2.0 ** -24 * mag
    assert np.all(np.abs(y - ref) <= bound), float(np.max(np.abs(y - ref) - bound))
    rounded = logits_f32(to_bf(ref.astype(np.float32))).reshape(n, rows)
    assert np.mean(y == rounded) > 0.99


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("n,rows,cols", [(1, 1, 128), (37, 70, 256), (130, 200, 2048), (256, 64, 4224),
                                         (300, 1100, 512), (33, 65, 48)])
def test_staged_matrix_gemm_bit_identical(n, rows, cols, mode):
    """The LDS-staged tiles the prefill runs (kernel 1) give the bits of the
    direct-fragment kernel (kernel 0) in every epilogue: same k-step rotation
    over the partial sums, same tree. Ragged token and row tails; widths that
    are not whole 128-column pairs of steps (48) run the direct kernel in the
    prefill too."""
    say("staged matrix gemm", n, rows, cols, "mode", mode)
    rng = np.random.default_rng(n * 7 + rows + cols + mode)
    x = to_bf(rng.standard_normal((n, cols)))
    w = to_bf(rng.standard_normal((rows, cols)) * 0.05)
    w2 = to_bf(rng.standard_normal((rows, cols)) * 0.05) if mode == 2 else None
    res = to_bf(rng.standard_normal((n, rows))) if mode == 1 else None
    a = device_gemm(x, w, w2, res, n, rows, cols, mode, 0)
    b = device_gemm(x, w, w2, res, n, rows, cols, mode, 1)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("name,n", [("mini", 37), ("mini-moe", 37), ("mini-moe", 300)])
@pytest.mark.parametrize("components", [Session.MATRIX_PROJECTIONS, Session.MATRIX_EXPERTS, ALL])
def test_matrix_prefill_within_reference_gate(name, n, components):
    cfg = shape(name)
    if not cfg["moe"] and components == Session.MATRIX_EXPERTS:
        pytest.skip("expert projections exist only in MoE models")
    say("matrix prefill", name, "tokens", n, "components", components)
    m = cq35.Model.synthetic(cfg, seed=9)
    prompt = np.random.default_rng(n).integers(0, cfg["vocab"], n).tolist()
    se, ce = prefill(m, prompt, 0, n + 8, decode=4)
    sm, cm = prefill(m, prompt, components, n + 8, decode=4)
    for i, ((te, le), (tm, lm)) in enumerate(zip(ce, cm)):
        r = rel_rms(logits_f32(lm), logits_f32(le))
        say(f"  call {i}: relative logit RMS {r:.4f}, tokens {te} / {tm}")
        assert np.all(np.isfinite(logits_f32(lm)))
        assert r <= 0.05, f"{name}: call {i} relative logit RMS {r:.4f} above the 5% gate"
    # the state the prompt leaves (KV rows, conv history, recurrent state)
    r = rel_rms(logits_f32(sm.export_state(0)), logits_f32(se.export_state(0)))
    say(f"  session state relative RMS {r:.4f}")
    assert r <= 0.05


@pytest.mark.parametrize("layers", [4, 40])
@pytest.mark.parametrize("components", [Session.MATRIX_PROJECTIONS, ALL, ALL | Session.MATRIX_ATTENTION])
def test_matrix_prefill_35b_within_exact_order_spread(layers, components):
    cfg = shape(f"qwen36-35b-a3b@{layers}")
    n, steps = 96, 3
    say("matrix prefill vs the exact orders' spread, 35B-A3B dims,", layers, "layers, tokens", n,
        "components", components)
    m = cq35.Model.synthetic(cfg, seed=9)
    prompt = np.random.default_rng(n).integers(0, cfg["vocab"], n).tolist()
    batched, per_token, matrix = m.session(n + 4), m.session(n + 4), m.session(n + 4)
    matrix.set_matrix_prefill(components)
    calls = [(batched.step_raw(prompt)[0], None, matrix.step_raw(prompt)[0])]
    for t in prompt:
        lt, _ = per_token.step_raw([t])
    calls[0] = (calls[0][0], lt, calls[0][2])
    # continue all three with the exact batched session's greedy tokens
    tok = int(np.argmax(logits_f32(calls[0][0])))
    for _ in range(steps):
        lb, nxt = batched.step_raw([tok])
        calls.append((lb, per_token.step_raw([tok])[0], matrix.step_raw([tok])[0]))
        tok = nxt
    for i, (lb, lt, lm) in enumerate(calls):
        assert np.all(np.isfinite(logits_f32(lm)))
        spread = rel_rms(logits_f32(lt), logits_f32(lb))
        r = rel_rms(logits_f32(lm), logits_f32(lb))
        say(f"  call {i}: exact orders differ by {spread:.4f}; matrix-core vs batched {r:.4f}")
        assert spread > 0.0
        assert r <= max(0.05, 1.25 * spread), f"call {i}: {r:.4f} outside the exact orders' spread {spread:.4f}"


def test_matrix_prefill_switch_leaves_decode_and_exact_path(oracle):
    cfg = cc.preset("mini-moe")
    m = cq35.Model.synthetic(cfg, seed=2)
    prompt = [5, 77, 901, 4096, 17]
    s = m.session(16)
    with pytest.raises(cq35.CQ35Error):
        s.set_matrix_prefill(8)
    s.set_matrix_prefill(ALL)
    s.set_matrix_prefill(0)
    logits, tok = s.step_raw(prompt)
    om = oracle.Model(cfg, oracle.synthetic_weights(cfg, 2))
    os_ = om.session(16)
    otok, ologits = os_.step(prompt, 0)
    assert tok == otok and np.array_equal(logits, ologits), "exact path changed by the switch"
    # decode steps are single-token calls: identical with the switch on
    a = m.session(16)
    b = m.session(16)
    b.set_matrix_prefill(ALL)
    ta = tb = 3
    for _ in range(6):
        la, ta = a.step_raw([ta])
        lb, tb = b.step_raw([tb])
        assert ta == tb and np.array_equal(la, lb)

"""Session checkpoints and the prompt prefix cache on the GPU, bitwise:
- tests/session_checkpoint.rs:112-168: a checkpoint taken after a 1024-token
  block resumes exactly like the cold session, also again after a resumed
  session decoded; another model rejects it;
- src/server/engine.rs:645-732 (serving_prefix_cache_bitwise_parity): warm
  prefills from the stable / recent checkpoints give the cold prefill's next
  token and logits bit for bit, a rewritten span falls back to the stable
  slot, another capacity misses, unrelated prompts and cancelled requests
  leave the slots alone.
On the reduced MoE shape (same code paths as 35B: batched prefill, persistent
decode)."""
import numpy as np
import pytest

import cq35
import cq35.config as cc
from cq35.prefix_cache import PrefixCache, prefill

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def model():
    return cq35.Model.synthetic(cc.preset("mini-moe"), seed=4)


def bits(logits):
    return np.asarray(logits, dtype=np.float32).view(np.uint32)


def test_checkpoint_resume_is_bitwise_exact_and_independent(model):
    say("checkpoint resume, 2051 tokens")
    tokens = [100 + i % 97 for i in range(2051)]
    s = model.session(4096)
    s.append_next_token(tokens[:1024])
    cp = s.into_checkpoint()
    assert cp.position == 1024 and cp.capacity == 4096 and cp.byte_len() > 0
    warm = model.resume_checkpoint(cp)
    warm.append_next_token(tokens[1024:2048])
    warm_logits = bits(warm.append_logits(tokens[2048:]))
    nxt = warm.decode_next_token(101)
    generated = [nxt]
    for _ in range(3):
        nxt = warm.decode_next_token(nxt)
        generated.append(nxt)
    del warm
    for label in ["cold", "restored again after decode"]:
        if label == "cold":
            s = model.session(4096)
            s.append_next_token(tokens[:1024])
        else:
            s = model.resume_checkpoint(cp)
        s.append_next_token(tokens[1024:2048])
        assert np.array_equal(bits(s.append_logits(tokens[2048:])), warm_logits), label
        nxt = s.decode_next_token(101)
        assert nxt == generated[0], label
        for expected in generated[1:]:
            nxt = s.decode_next_token(nxt)
            assert nxt == expected, label
    other = cq35.Model.synthetic(cc.preset("mini-moe"), seed=4)
    with pytest.raises(ValueError):
        other.resume_checkpoint(cp)


def test_serving_prefix_cache_bitwise_parity(model):
    say("prefix cache parity")
    cancel = {"now": False}
    cancelled = lambda: cancel["now"]
    cache = PrefixCache()
    tokens = [100 + i % 97 for i in range(2051)]

    def cold(toks, capacity):
        s, nxt, _, _ = prefill(model, PrefixCache(), False, toks, capacity, 1024)
        return nxt, bits(s.decode_logits(nxt))

    # both slots, including the exact-checkpoint / no-suffix path
    for enabled, expected in [(True, 0), (True, 2048), (False, 0)]:
        s, nxt, cached, _ = prefill(model, cache, enabled, tokens[:2048], 4096, 1024, cancelled)
        assert cached == expected
        logits = bits(s.decode_logits(nxt))
        cnext, clogits = cold(tokens[:2048], 4096)
        assert nxt == cnext and np.array_equal(logits, clogits)
    # mutating a restored decode session above must leave the prompt frozen
    for end, changed, capacity, expected in [(2049, False, 4096, 2048), (2051, False, 4096, 2048),
                                             (2051, True, 4096, 1024), (2051, False, 8192, 0)]:
        if changed:
            tokens[1400] += 1  # rewritten earlier reasoning
        s, nxt, cached, _ = prefill(model, cache, True, tokens[:end], capacity, 1024, cancelled)
        assert cached == expected, (end, changed, capacity)
        logits = bits(s.decode_logits(nxt))
        del s
        cnext, clogits = cold(tokens[:end], capacity)
        assert nxt == cnext and np.array_equal(logits, clogits)
    # unrelated short prompts and cancelled requests leave both slots intact
    stable, recent = cache.stable, cache.recent
    prefill(model, cache, True, [1, 2, 3], 16, 0, cancelled)
    assert cache.stable is stable and cache.recent is recent
    cancel["now"] = True
    assert prefill(model, cache, True, tokens, 8192, 1024, cancelled) is None
    cancel["now"] = False
    cache.clear()
    _, _, cached, _ = prefill(model, cache, True, tokens, 8192, 1024, cancelled)
    assert cached == 0

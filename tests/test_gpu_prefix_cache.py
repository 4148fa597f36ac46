"""Session checkpoints on the GPU, bitwise, as the serving loop's prompt
prefix cache uses them through this ABI (the cache policy itself stays in the
Rust server, src/server/prefix_cache.rs):
- tests/session_checkpoint.rs:112-168: a checkpoint taken after a 1024-token
  block resumes exactly like the cold session, also again after a resumed
  session decoded; another model rejects it;
- resume equals cold at every absolute block boundary a server can hold
  (1024 and 2048 tokens), with and without a suffix to prefill: the warm
  prefill gives the cold prefill's next token and logits bit for bit, the
  checkpoint stays frozen while sessions resumed from it decode, and a
  checkpoint is only valid for its own capacity.
On the reduced MoE shape (same code paths as 35B: batched prefill, persistent
decode)."""
import numpy as np
import pytest

import cq35
import cq35.config as cc

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


def test_resume_equals_cold_at_block_boundaries(model):
    say("resume equals cold at 1024-token block boundaries")
    tokens = [100 + (7 * i) % 97 for i in range(2051)]

    def prefill(s, start, end):
        """The prompt from `start` in absolute 1024-token blocks."""
        nxt = None
        for b in range(start, end, 1024):
            nxt = s.append_next_token(tokens[b:min(b + 1024, end)])
        return nxt

    base = model.session(4096)
    after = {1024: prefill(base, 0, 1024)}  # next token of the prompt ending at the checkpoint
    cp1024 = base.into_checkpoint()
    s = model.resume_checkpoint(cp1024)
    after[2048] = prefill(s, 1024, 2048)
    cp2048 = s.into_checkpoint()
    for end in (1024, 2048, 2049, 2051):
        c = model.session(4096)
        cnext = prefill(c, 0, end)
        clogits = bits(c.decode_logits(cnext))
        cfollow = c.decode_next_token(cnext)
        del c
        for cp in (cp1024, cp2048):
            if cp.position > end:
                continue
            say("  prompt", end, "from checkpoint", cp.position)
            s = model.resume_checkpoint(cp)
            # an exact checkpoint has nothing left to prefill
            nxt = prefill(s, cp.position, end) if end > cp.position else after[cp.position]
            assert nxt == cnext, (end, cp.position)
            assert np.array_equal(bits(s.decode_logits(nxt)), clogits), (end, cp.position)
            # decoding on the resumed session leaves the checkpoint as it was
            # (later resumes of the same checkpoint are compared again)
            assert s.decode_next_token(nxt) == cfollow, (end, cp.position)
            assert s.capacity == cp.capacity == 4096

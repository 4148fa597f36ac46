"""Prompt prefix cache of the serving loop (src/server/prefix_cache.rs and
the prefill of src/server/engine.rs:273-377), over this library's session
checkpoints.

Two immutable checkpoints: `stable` (the end of the conversation prefix the
caller marks stable, rounded down to a block) and `recent` (the last block
boundary of the latest prompt). Prompts are prefilled in absolute blocks of
PREFILL_BLOCK tokens, so a request that resumes from a checkpoint runs the
same multi-token calls as a cold one: results are bitwise identical (the F32
recurrent state round-trips through BF16 at every call boundary, so the
block boundaries must match). A session is never rewound by changing its
position: DeltaNet state cannot be rewound that way.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Callable, Optional, Sequence

PREFILL_BLOCK = 1024


@dataclass(frozen=True)
class Entry:
    tokens: tuple
    capacity: int
    state: Any = field(compare=False)
    next: int = 0


class PrefixCache:
    def __init__(self):
        self.stable: Optional[Entry] = None
        self.recent: Optional[Entry] = None

    def clear(self) -> None:
        self.stable = None
        self.recent = None

    def matching(self, tokens: Sequence[int], capacity: int, limit: int) -> Optional[Entry]:
        """The longest slot whose tokens prefix `tokens`, with the same
        capacity and at most `limit` tokens (prefix_cache.rs:33-43)."""
        best = None
        for e in (self.stable, self.recent):
            if (e is not None and e.capacity == capacity and len(e.tokens) <= limit
                    and tuple(tokens[:len(e.tokens)]) == e.tokens):
                if best is None or len(e.tokens) > len(best.tokens):
                    best = e
        return best

    def exact(self, tokens: Sequence[int], capacity: int) -> Optional[Entry]:
        e = self.matching(tokens, capacity, len(tokens))
        return e if e is not None and len(e.tokens) == len(tokens) else None


def block_boundary(position: int) -> int:
    return position // PREFILL_BLOCK * PREFILL_BLOCK


def common_prefix(left: Sequence[int], right: Sequence[int]) -> int:
    n = 0
    for a, b in zip(left, right):
        if a != b:
            break
        n += 1
    return n


def capacity_bucket(required: int, context: int) -> int:
    """The next power of two at or above `required`, at most `context`."""
    if required <= 1:
        return min(1, context)
    return min(1 << (required - 1).bit_length(), context)


def prefill(model, cache: PrefixCache, enabled: bool, tokens: Sequence[int], capacity: int,
            stable: int, cancelled: Callable[[], bool] = lambda: False):
    """Prefill `tokens` (engine.rs:273-377): resume from the longest matching
    checkpoint, append the rest in absolute PREFILL_BLOCK blocks, and write
    checkpoints through at the stable and recent boundaries. Returns
    (session, next token, cached tokens, tokens written to the cache), or
    None when cancelled."""
    if cancelled():
        return None
    tokens = list(tokens)
    recent = block_boundary(len(tokens))
    # a new stable checkpoint must not be jumped past
    limit = stable if stable > 0 and cache.exact(tokens[:stable], capacity) is None else len(tokens)
    hit = cache.matching(tokens, capacity, limit) if enabled else None
    session, nxt, cached = None, 0, 0
    if hit is not None:
        try:
            session = model.resume_checkpoint(hit.state)
            cached = len(hit.tokens)
            nxt = hit.next
            if cached == stable:
                cache.stable = hit
            if cached == recent:
                cache.recent = hit
        except Exception:
            cache.clear()
            session = None
    if session is None:
        session, nxt, cached = model.session(capacity), 0, 0
    written = cached
    while session.position < len(tokens):
        if cancelled():
            return None
        pos = session.position
        end = min((pos // PREFILL_BLOCK + 1) * PREFILL_BLOCK, len(tokens))
        nxt = session.append_next_token(tokens[pos:end])
        if cancelled():
            return None
        if enabled and end > 0 and (end == stable or end == recent):
            entry = cache.exact(tokens[:end], capacity)
            if entry is None:
                # evict first: at most two snapshots plus one live session
                if end == stable:
                    cache.stable = None
                if end == recent:
                    cache.recent = None
                entry = Entry(tuple(tokens[:end]), capacity, session.into_checkpoint(), nxt)
                session = model.resume_checkpoint(entry.state)
                written = end
            if end == stable:
                cache.stable = entry
            if end == recent:
                cache.recent = entry
    return session, nxt, cached, written - cached

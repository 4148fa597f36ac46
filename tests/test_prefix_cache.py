"""The prefix cache's slot policy and block arithmetic on the CPU: the
reference's own unit tests (src/server/prefix_cache.rs:66-114), same cases
and answers."""
from cq35.prefix_cache import Entry, PrefixCache, block_boundary, capacity_bucket, common_prefix


def entry(tokens, capacity):
    return Entry(tuple(tokens), capacity, None, 42)


def test_longest_exact_token_prefix_with_same_capacity_only():
    cache = PrefixCache()
    cache.stable = entry([1, 2], 8)
    cache.recent = entry([1, 2, 3, 4], 8)
    assert len(cache.matching([1, 2, 3, 4, 5], 8, 5).tokens) == 4
    # a rewritten reasoning span invalidates the recent slot, not the stable one
    assert len(cache.matching([1, 2, 9, 4, 5], 8, 5).tokens) == 2
    assert cache.matching([1, 7, 3, 4], 8, 4) is None
    assert cache.matching([1, 2, 3, 4], 16, 4) is None
    assert cache.matching([1], 8, 1) is None
    assert cache.exact([1, 2, 3, 4], 8).next == 42
    assert cache.exact([1, 2, 3], 8) is None
    assert len(cache.matching([1, 2, 3, 4], 8, 2).tokens) == 2
    cache.clear()
    assert cache.matching([1, 2], 8, 2) is None


def test_absolute_blocks_and_capacity_buckets():
    assert block_boundary(1023) == 0
    assert block_boundary(1024) == 1024
    assert block_boundary(2050) == 2048
    assert common_prefix([1, 2, 3], [1, 2, 4]) == 2
    assert capacity_bucket(1024, 5000) == 1024
    assert capacity_bucket(1025, 5000) == 2048
    assert capacity_bucket(4097, 5000) == 5000
    top = 2 ** 64 - 1
    assert capacity_bucket(top, top) == top

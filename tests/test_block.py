"""Block pool behaviour: the reference's allocator tests (tests/test_block.py:6-77)
restated on BlockPool, plus random operation sequences checked step by step
against a direct model of the reference allocator (vllmlite/block.py:45-138):
the same block ids handed out and the same free count after every operation."""

from collections import OrderedDict

import numpy as np
import pytest

from vllmlite_amd.kvpool import BlockPool, OutOfBlocks, chain_digest


def test_alloc_and_free_roundtrip():
    p = BlockPool(4, 16, prefix_caching=False)
    ids = [p.allocate() for _ in range(4)]
    assert len(set(ids)) == 4 and p.num_free == 0
    with pytest.raises(OutOfBlocks):
        p.allocate()
    for i in ids:
        p.release(i)
    assert p.num_free == 4


def test_fresh_ids_are_lifo():
    p = BlockPool(4, 16, prefix_caching=False)
    assert [p.allocate(), p.allocate()] == [3, 2]
    p.release(3)
    assert p.allocate() == 3


def test_refcount_holds_block():
    p = BlockPool(2, 16, prefix_caching=False)
    b = p.allocate()
    p.share(b)
    assert p.is_shared(b)
    p.release(b)
    assert not p.is_shared(b) and p.num_free == 1
    p.release(b)
    assert p.num_free == 2


def test_double_free_raises():
    p = BlockPool(1, 16)
    b = p.allocate()
    p.release(b)
    with pytest.raises(ValueError):
        p.release(b)


def test_full_block_is_shareable_while_still_in_use():
    p = BlockPool(4, 4)
    b = p.allocate()
    d = chain_digest(None, (1, 2, 3, 4))
    p.publish(b, d)
    assert p.lookup(d) == b and p.refs[b] == 2


def test_cached_block_is_evictable_once_unreferenced():
    p = BlockPool(2, 4)
    b = p.allocate()
    p.publish(b, chain_digest(None, (1, 2, 3, 4)))
    p.release(b)
    assert p.num_free == 2
    assert {p.allocate(), p.allocate()} == {0, 1}
    assert p.lookup(chain_digest(None, (1, 2, 3, 4))) is None  # evicted


def test_digest_chains_the_prefix():
    d1 = chain_digest(None, (1, 2))
    assert chain_digest(d1, (3, 4)) != chain_digest(chain_digest(None, (9, 9)), (3, 4))
    assert chain_digest(None, (1, 2)) == d1 and chain_digest(None, (2, 1)) != d1


def test_hit_rate_tracking():
    p = BlockPool(4, 4)
    d = chain_digest(None, (1, 2, 3, 4))
    b = p.allocate()
    p.publish(b, d)
    assert p.lookup(d) == b
    assert p.stats()["prefix_hit_rate"] == 1.0 and p.stats()["cached_blocks"] == 1


class _ModelAllocator:
    """The reference allocator's algorithm, written directly: a free-id list
    popped from the end, refcounts, a content hash per block and an ordered
    hash -> block map whose free count is a scan."""

    def __init__(self, n, prefix):
        self.prefix = prefix
        self.ref = [0] * n
        self.h = [None] * n
        self.free_ids = list(range(n))
        self.cached = OrderedDict()

    @property
    def num_free(self):
        return len(self.free_ids) + sum(1 for b in self.cached.values() if self.ref[b] == 0)

    def allocate(self):
        if self.free_ids:
            b = self.free_ids.pop()
        else:
            for h, b in self.cached.items():
                if self.ref[b] == 0:
                    self.cached.pop(h)
                    self.h[b] = None
                    break
            else:
                raise OutOfBlocks()
        self.ref[b] = 1
        self.h[b] = None
        return b

    def free(self, b):
        self.ref[b] -= 1
        if self.ref[b]:
            return
        if self.prefix and self.h[b] is not None:
            self.cached[self.h[b]] = b
            self.cached.move_to_end(self.h[b])
        else:
            self.free_ids.append(b)

    def mark_full(self, b, h):
        if not self.prefix or self.h[b] == h:
            return
        self.h[b] = h
        self.cached[h] = b
        self.cached.move_to_end(h)

    def reuse(self, h):
        b = self.cached.get(h)
        if b is None:
            return None
        self.cached.move_to_end(h)
        self.ref[b] += 1
        return b


@pytest.mark.parametrize("trial", range(24))
def test_pool_matches_the_reference_allocator_model(trial):
    """Random allocate / share / release / publish / reuse sequences with a
    few distinct digests, so blocks collide on a digest (entries re-pointed,
    stale blocks not counted free) and blocks get re-published."""
    rng = np.random.default_rng(trial)
    prefix = trial % 4 != 0
    n = 10
    pool, model = BlockPool(n, 4, prefix), _ModelAllocator(n, prefix)
    digests = [chain_digest(None, (k,)) for k in range(4)]
    held = []
    for _ in range(500):
        op = int(rng.integers(0, 5))
        if op == 0:
            try:
                want = model.allocate()
            except OutOfBlocks:
                with pytest.raises(OutOfBlocks):
                    pool.allocate()
            else:
                assert pool.allocate() == want
                held.append(want)
        elif op == 1 and held:
            b = held.pop(int(rng.integers(0, len(held))))
            pool.release(b)
            model.free(b)
        elif op == 2 and held:
            b = held[int(rng.integers(0, len(held)))]
            pool.share(b)
            model.ref[b] += 1
            held.append(b)
        elif op == 3 and held:
            b = held[int(rng.integers(0, len(held)))]
            d = digests[int(rng.integers(0, 4))]
            pool.publish(b, d)
            model.mark_full(b, d)
        elif op == 4 and prefix:
            d = digests[int(rng.integers(0, 4))]
            got, want = pool.lookup(d), model.reuse(d)
            assert got == want
            if got is not None:
                held.append(got)
        assert pool.num_free == model.num_free
        assert pool.refs == model.ref
        assert list(pool.index.items()) == list(model.cached.items())
        assert pool.audit()

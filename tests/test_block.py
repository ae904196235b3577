"""Allocator behaviour (the reference's tests/test_block.py:6-77) plus the
exactness of the running free-block count against the reference's scan."""

import numpy as np
import pytest

from vllmlite_amd.block import BlockAllocator, OutOfBlocks, hash_block


def test_alloc_and_free_roundtrip():
    a = BlockAllocator(4, 16, enable_prefix_caching=False)
    ids = [a.allocate()[0] for _ in range(4)]
    assert len(set(ids)) == 4 and a.num_free == 0
    with pytest.raises(OutOfBlocks):
        a.allocate()
    for i in ids:
        a.free(i)
    assert a.num_free == 4


def test_fresh_ids_are_lifo():
    a = BlockAllocator(4, 16, enable_prefix_caching=False)
    assert [a.allocate()[0] for _ in range(2)] == [3, 2]
    a.free(3)
    assert a.allocate()[0] == 3


def test_refcount_holds_block():
    a = BlockAllocator(2, 16, enable_prefix_caching=False)
    bid, _ = a.allocate()
    a.fork(bid)
    assert a.is_shared(bid)
    a.free(bid)
    assert not a.is_shared(bid) and a.num_free == 1
    a.free(bid)
    assert a.num_free == 2


def test_double_free_raises():
    a = BlockAllocator(1, 16)
    bid, _ = a.allocate()
    a.free(bid)
    with pytest.raises(ValueError):
        a.free(bid)


def test_full_block_is_shareable_while_still_in_use():
    a = BlockAllocator(4, 4)
    bid, hit = a.allocate()
    assert not hit
    h = hash_block(None, (1, 2, 3, 4))
    a.mark_full(bid, h)
    same, hit2 = a.allocate(h)
    assert hit2 and same == bid and a.blocks[bid].ref_count == 2


def test_cached_block_is_evictable_once_unreferenced():
    a = BlockAllocator(2, 4)
    b1, _ = a.allocate()
    a.mark_full(b1, hash_block(None, (1, 2, 3, 4)))
    a.free(b1)
    assert a.num_free == 2
    assert {a.allocate()[0], a.allocate()[0]} == {0, 1}


def test_hash_chains_the_prefix():
    h1 = hash_block(None, (1, 2))
    assert hash_block(h1, (3, 4)) != hash_block(hash_block(None, (9, 9)), (3, 4))


def test_hash_is_blake2b_of_the_documented_bytes():
    import hashlib
    want = hashlib.blake2b(b"|1,2,3", digest_size=16).hexdigest()
    assert hash_block(None, (1, 2, 3)) == want
    want2 = hashlib.blake2b((want + "|4").encode(), digest_size=16).hexdigest()
    assert hash_block(want, (4,)) == want2


def test_hit_rate_tracking():
    a = BlockAllocator(4, 4)
    h = hash_block(None, (1, 2, 3, 4))
    bid, _ = a.allocate(h)
    a.mark_full(bid, h)
    a.allocate(h)
    assert a.stats()["prefix_hit_rate"] == 0.5


def test_running_free_count_equals_the_scan_under_random_ops():
    """Random allocate/fork/free/mark_full, including hash collisions between
    blocks (overwritten map entries) and re-publishing under a new hash."""
    rng = np.random.default_rng(0)
    for trial in range(20):
        a = BlockAllocator(12, 4, enable_prefix_caching=bool(trial % 4))
        held = []
        for _ in range(400):
            op = rng.integers(0, 5)
            try:
                if op == 0:
                    h = None if rng.random() < 0.5 else hash_block(None, (int(rng.integers(0, 4)),))
                    bid, _ = a.allocate(h)
                    held.append(bid)
                elif op == 1 and held:
                    a.free(held.pop(int(rng.integers(0, len(held)))))
                elif op == 2 and held:
                    bid = held[int(rng.integers(0, len(held)))]
                    a.fork(bid)
                    held.append(bid)
                elif op == 3 and held:
                    bid = held[int(rng.integers(0, len(held)))]
                    a.mark_full(bid, hash_block(None, (int(rng.integers(0, 4)),)))
                elif op == 4:
                    a.take_cached(hash_block(None, (int(rng.integers(0, 4)),))) is not None and None
            except OutOfBlocks:
                pass
            assert a.check_counts()

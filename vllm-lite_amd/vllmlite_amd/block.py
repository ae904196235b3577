"""Physical KV block bookkeeping: refcounts, a LIFO free list, and an LRU map
of published (hashed) blocks for prefix reuse.

Behaviour follows vllmlite/block.py:16-156, because physical block ids decide
every flat cache slot the kernels touch:

* fresh ids come off the END of a free list that starts as 0..n-1 and gets
  freed ids appended (block.py:57, 71-72, 114);
* when the free list is empty, the coldest entry of the hash map whose block
  is unreferenced is evicted (block.py:74-79);
* a freed block with a content hash stays in the hash map instead of going back
  on the free list (block.py:109-112).

One thing is implemented differently. `num_free` (block.py:63-68) scans the
whole hash map and counts entries whose block is unreferenced; it runs inside
every `can_allocate`. Here an exact running count of such entries is kept
instead: `_entries[bid]` counts hash-map entries that point at `bid` (an entry
can be overwritten when two blocks publish the same hash, and a block can be
left behind under an old hash), and `_evictable` is the sum of `_entries[bid]`
over blocks with refcount 0. Every write to the map or to a refcount goes
through the helpers below, and `check_counts()` recomputes the reference's
scan so tests can assert the two agree.
"""

from __future__ import annotations

import hashlib
from collections import OrderedDict
from dataclasses import dataclass, field
from typing import List, Optional, Tuple


class OutOfBlocks(Exception):
    pass


@dataclass
class Block:
    block_id: int
    ref_count: int = 0
    content_hash: Optional[str] = None
    num_tokens: int = 0

    @property
    def is_free(self) -> bool:
        return self.ref_count == 0


def hash_block(prev_hash: Optional[str], token_ids: Tuple[int, ...]) -> str:
    """Chained 128-bit BLAKE2b over the previous block's hex digest, a "|"
    separator and the comma-joined decimal token ids (block.py:34-40). The
    digest decides prefix-cache hits, so the byte string hashed is the same."""
    h = hashlib.blake2b(digest_size=16)
    if prev_hash:
        h.update(prev_hash.encode())
    h.update(b"|")
    h.update(",".join(map(str, token_ids)).encode())
    return h.hexdigest()


class BlockAllocator:
    def __init__(self, num_blocks: int, block_size: int, enable_prefix_caching: bool = True):
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.enable_prefix_caching = enable_prefix_caching
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.free_ids: List[int] = list(range(num_blocks))
        self.cached: "OrderedDict[str, int]" = OrderedDict()
        self.hits = 0
        self.misses = 0
        self._entries = [0] * num_blocks
        self._evictable = 0

    # -- exact bookkeeping of "cached entries whose block is unreferenced" --

    def _map_set(self, h: str, bid: int) -> None:
        old = self.cached.get(h)
        if old is not None:
            self._entries[old] -= 1
            if self.blocks[old].ref_count == 0:
                self._evictable -= 1
        self.cached[h] = bid
        self._entries[bid] += 1
        if self.blocks[bid].ref_count == 0:
            self._evictable += 1

    def _map_pop(self, h: str) -> int:
        bid = self.cached.pop(h)
        self._entries[bid] -= 1
        if self.blocks[bid].ref_count == 0:
            self._evictable -= 1
        return bid

    def _set_ref(self, blk: Block, value: int) -> None:
        n = self._entries[blk.block_id]
        if n:
            was_free = blk.ref_count == 0
            now_free = value == 0
            if was_free and not now_free:
                self._evictable -= n
            elif now_free and not was_free:
                self._evictable += n
        blk.ref_count = value

    def check_counts(self) -> bool:
        """True when the running count equals block.py:67's scan."""
        scan = sum(1 for bid in self.cached.values() if self.blocks[bid].is_free)
        return scan == self._evictable

    # -- the reference's interface --

    @property
    def num_free(self) -> int:
        return len(self.free_ids) + self._evictable

    def _take_free_id(self) -> int:
        if self.free_ids:
            return self.free_ids.pop()
        victim = None
        for h, bid in self.cached.items():
            if self.blocks[bid].ref_count == 0:
                victim = h
                break
        if victim is None:
            raise OutOfBlocks("no blocks left")
        bid = self._map_pop(victim)
        self.blocks[bid].content_hash = None
        return bid

    def allocate(self, content_hash: Optional[str] = None) -> Tuple[int, bool]:
        """Returns (block_id, was_cache_hit) (block.py:81-97)."""
        if self.enable_prefix_caching and content_hash is not None:
            bid = self.cached.get(content_hash)
            if bid is not None:
                self.cached.move_to_end(content_hash)
                blk = self.blocks[bid]
                self._set_ref(blk, blk.ref_count + 1)
                self.hits += 1
                return bid, True
            self.misses += 1
        bid = self._take_free_id()
        blk = self.blocks[bid]
        self._set_ref(blk, 1)
        blk.num_tokens = 0
        blk.content_hash = None
        return bid, False

    def take_cached(self, content_hash: str) -> Optional[int]:
        """Prefix-reuse lookup used by BlockManager.reuse_prefix
        (block_manager.py:50-56): on a hit, touch the LRU order, add a
        reference and count a hit. Returns None on a miss (no miss counted)."""
        bid = self.cached.get(content_hash)
        if bid is None:
            return None
        self.cached.move_to_end(content_hash)
        blk = self.blocks[bid]
        self._set_ref(blk, blk.ref_count + 1)
        self.hits += 1
        return bid

    def fork(self, block_id: int) -> None:
        blk = self.blocks[block_id]
        self._set_ref(blk, blk.ref_count + 1)

    def free(self, block_id: int) -> None:
        blk = self.blocks[block_id]
        if blk.ref_count == 0:
            raise ValueError(f"double free on block {block_id}")
        self._set_ref(blk, blk.ref_count - 1)
        if blk.ref_count:
            return
        if self.enable_prefix_caching and blk.content_hash is not None:
            self._map_set(blk.content_hash, block_id)
            self.cached.move_to_end(blk.content_hash)
        else:
            self.free_ids.append(block_id)

    def mark_full(self, block_id: int, content_hash: str) -> None:
        """Publish a block as soon as it fills (block.py:116-129)."""
        blk = self.blocks[block_id]
        blk.num_tokens = self.block_size
        if not self.enable_prefix_caching or blk.content_hash == content_hash:
            return
        blk.content_hash = content_hash
        self._map_set(content_hash, block_id)
        self.cached.move_to_end(content_hash)

    def is_shared(self, block_id: int) -> bool:
        return self.blocks[block_id].ref_count > 1

    def stats(self) -> dict:
        used = self.num_blocks - self.num_free
        total = self.hits + self.misses
        return {
            "blocks_total": self.num_blocks,
            "blocks_used": used,
            "usage": used / self.num_blocks,
            "cached_blocks": len(self.cached),
            "prefix_hit_rate": self.hits / total if total else 0.0,
        }


@dataclass
class BlockTable:
    """Logical -> physical block mapping of one sequence."""

    block_ids: List[int] = field(default_factory=list)
    num_filled: int = 0

    def slot(self, block_size: int, pos: int) -> int:
        """Flat cache slot of token position `pos` (block.py:154-156)."""
        return self.block_ids[pos // block_size] * block_size + pos % block_size

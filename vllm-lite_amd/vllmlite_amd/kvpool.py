"""The paged KV block pool: refcounted physical blocks, a LIFO stack of fresh
blocks and a prefix index of published full blocks.

Behaviour pinned by the reference (vllmlite/block.py:45-138) and by its
published step counts, which depend on it:

  * a fresh block is the most recently returned one (LIFO); blocks start
    numbered so that the first allocations are n-1, n-2, ...;
  * a block that fills up is published under the digest of its contents and
    of every block before it, the moment it fills (block.py:115-128); a block
    whose last reference goes away stays indexed (and allocatable again) if
    it is published, else it returns to the stack (block.py:103-113);
  * when the stack is empty the coldest indexed block with no references is
    evicted (block.py:69-78); the index is ordered coldest first and a block
    moves to the warm end when it is published, freed or reused;
  * one digest maps to one block: publishing or freeing a block under a digest
    that already maps to another block re-points the entry, and the other
    block, still carrying that digest, is then reachable by no lookup and is
    not counted free (block.py:64-67 counts index entries);
  * the free count is the fresh stack plus the index entries whose block has
    no references (block.py:63-67).

Design: per-block state in flat Python lists (refcount, digest, index
entries pointing at it), the index an OrderedDict digest -> block, and the
free count kept exactly by updating it on every refcount or index change
instead of scanning the index. Digests are 16-byte BLAKE2b over the parent
block's digest and the block's token ids as little-endian int32, computed
once per block when it fills (incremental: a block extends its parent's
digest).
"""

from __future__ import annotations

import hashlib
from collections import OrderedDict
from typing import List, Optional

import numpy as np


class OutOfBlocks(Exception):
    """No fresh block and no evictable published block (block.py:16-17, 78)."""


def chain_digest(parent: Optional[bytes], tokens) -> bytes:
    """Digest of a full block: its parent's digest (empty for the first block)
    followed by the block's token ids as little-endian int32."""
    h = hashlib.blake2b(digest_size=16)
    if parent is not None:
        h.update(parent)
    h.update(np.asarray(tokens, dtype="<i4").tobytes())
    return h.digest()


class BlockList:
    """A request's block table: physical block ids in position order and the
    number of token slots whose K/V is written (vllmlite/block.py:142-156)."""

    __slots__ = ("block_ids", "num_filled")

    def __init__(self, block_ids: Optional[List[int]] = None, num_filled: int = 0):
        self.block_ids = block_ids if block_ids is not None else []
        self.num_filled = num_filled

    def slot(self, block_size: int, pos: int) -> int:
        return self.block_ids[pos // block_size] * block_size + pos % block_size


class BlockPool:
    def __init__(self, num_blocks: int, block_size: int, prefix_caching: bool = True):
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.prefix_caching = prefix_caching
        self.refs = [0] * num_blocks
        self.digest: List[Optional[bytes]] = [None] * num_blocks
        self.entries = [0] * num_blocks  # index entries that point at the block
        self.fresh = list(range(num_blocks))  # pop() hands out the highest id first
        self.index: "OrderedDict[bytes, int]" = OrderedDict()
        self._evictable = 0  # index entries whose block has no reference
        self.hits = 0
        self.misses = 0

    # ---------------------------------------------------------------- counts --
    @property
    def num_free(self) -> int:
        return len(self.fresh) + self._evictable

    def is_shared(self, b: int) -> bool:
        return self.refs[b] > 1

    # ------------------------------------------------------- refcount changes --
    def _ref(self, b: int) -> None:
        if self.refs[b] == 0:
            self._evictable -= self.entries[b]
        self.refs[b] += 1

    def _point(self, d: bytes, b: int) -> None:
        """index[d] = b, moved to the warm end."""
        old = self.index.get(d)
        if old is not None:
            self.entries[old] -= 1
            if self.refs[old] == 0:
                self._evictable -= 1
        self.index[d] = b
        self.index.move_to_end(d)
        self.entries[b] += 1
        if self.refs[b] == 0:
            self._evictable += 1

    # ------------------------------------------------------------- operations --
    def allocate(self) -> int:
        """A block for new tokens: fresh if any, else the coldest evictable
        published block, which loses its digest."""
        if self.fresh:
            b = self.fresh.pop()
        else:
            for d, b in self.index.items():
                if self.refs[b] == 0:
                    break
            else:
                raise OutOfBlocks("no blocks left")
            del self.index[d]
            self.entries[b] -= 1
            self._evictable -= 1
            self.digest[b] = None
        self._ref(b)
        self.digest[b] = None
        return b

    def share(self, b: int) -> None:
        """One more holder of a held block (a forked request)."""
        self._ref(b)

    def lookup(self, d: bytes) -> Optional[int]:
        """Reuse the published block with digest d, if any: it gains a
        reference and moves to the warm end (block_manager.py:49-56)."""
        b = self.index.get(d)
        if b is None:
            return None
        self.index.move_to_end(d)
        self._ref(b)
        self.hits += 1
        return b

    def release(self, b: int) -> None:
        r = self.refs[b]
        if r == 0:
            raise ValueError(f"double free on block {b}")
        self.refs[b] = r - 1
        if r > 1:
            return
        self._evictable += self.entries[b]
        d = self.digest[b]
        if self.prefix_caching and d is not None:
            self._point(d, b)
        else:
            self.fresh.append(b)

    def publish(self, b: int, d: bytes) -> None:
        """Block b just filled: index it under digest d (block.py:115-128)."""
        if not self.prefix_caching or self.digest[b] == d:
            return
        self.digest[b] = d
        self._point(d, b)

    # ------------------------------------------------------------ diagnostics --
    def audit(self) -> bool:
        """The incremental free count equals a scan of the index."""
        scan = sum(1 for b in self.index.values() if self.refs[b] == 0)
        ent = [0] * self.num_blocks
        for b in self.index.values():
            ent[b] += 1
        return scan == self._evictable and ent == self.entries and all(r >= 0 for r in self.refs)

    def stats(self) -> dict:
        used = self.num_blocks - self.num_free
        looked = self.hits + self.misses
        return {
            "blocks_total": self.num_blocks,
            "blocks_used": used,
            "usage": used / self.num_blocks,
            "cached_blocks": len(self.index),
            "prefix_hit_rate": self.hits / looked if looked else 0.0,
        }

    def prefix_digests(self, tokens, count: int) -> List[bytes]:
        """Digests of the first `count` full blocks of a token list."""
        bs, out, d = self.block_size, [], None
        for i in range(count):
            d = chain_digest(d, tokens[i * bs:(i + 1) * bs])
            out.append(d)
        return out


def blocks_for(tokens: int, block_size: int) -> int:
    return -(-tokens // block_size)


__all__ = ["BlockList", "BlockPool", "OutOfBlocks", "blocks_for", "chain_digest"]


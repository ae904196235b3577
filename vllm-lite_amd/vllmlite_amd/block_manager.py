"""Grows sequences' block tables, emits copy-on-write pairs and publishes full
blocks for prefix reuse. Behaviour follows vllmlite/block_manager.py:16-153.

The CoW pairs returned by `append_slots` are what the copy-blocks kernel
consumes; the block tables are what the attention kernel follows.
"""

from __future__ import annotations

from typing import List, Optional, Tuple

from .block import BlockAllocator, BlockTable, hash_block
from .config import CacheConfig


class BlockManager:
    def __init__(self, cfg: CacheConfig):
        self.block_size = cfg.block_size
        self.allocator = BlockAllocator(cfg.num_blocks, cfg.block_size, cfg.enable_prefix_caching)
        self.prefix_caching = cfg.enable_prefix_caching
        self.peak_blocks = 0
        self.live_tokens = 0
        self.peak_live_tokens = 0

    def _blocks_needed(self, num_tokens: int) -> int:
        return -(-num_tokens // self.block_size)

    def can_allocate(self, seq, num_new_tokens: int, watermark_blocks: int = 0) -> bool:
        filled = seq.table.num_filled
        extra = self._blocks_needed(filled + num_new_tokens) - self._blocks_needed(filled)
        return self.allocator.num_free >= extra + watermark_blocks

    def reuse_prefix(self, seq) -> int:
        """Attach cached full blocks matching the prompt prefix; returns the
        number of prompt tokens skipped (block_manager.py:32-63). At least one
        prompt token is always left to run so the step yields logits."""
        if not self.prefix_caching or seq.table.block_ids:
            return 0
        bs = self.block_size
        toks = seq.prompt_token_ids
        prev: Optional[str] = None
        reused = 0
        for i in range((len(toks) - 1) // bs):
            h = hash_block(prev, tuple(toks[i * bs:(i + 1) * bs]))
            bid = self.allocator.take_cached(h)
            if bid is None:
                break
            seq.table.block_ids.append(bid)
            prev = h
            reused += bs
        seq.table.num_filled = reused
        seq.num_computed = reused
        seq.cached_prefix_tokens = reused
        return reused

    def append_slots(self, seq, num_new_tokens: int) -> List[Tuple[int, int]]:
        """Make room for num_new_tokens; return (src, dst) CoW pairs the runner
        must copy before any K/V write (block_manager.py:65-93)."""
        cows: List[Tuple[int, int]] = []
        table = seq.table
        bs = self.block_size
        alloc = self.allocator
        if table.num_filled % bs:
            idx = table.num_filled // bs
            if idx < len(table.block_ids):
                tail = table.block_ids[idx]
                if alloc.is_shared(tail):
                    new_id, _ = alloc.allocate()
                    cows.append((tail, new_id))
                    alloc.free(tail)
                    table.block_ids[idx] = new_id
        target = table.num_filled + num_new_tokens
        while len(table.block_ids) * bs < target:
            bid, _ = alloc.allocate()
            table.block_ids.append(bid)
        used = alloc.num_blocks - alloc.num_free
        if used > self.peak_blocks:
            self.peak_blocks = used
        return cows

    def slot_mapping(self, seq, start: int, count: int) -> List[int]:
        return [seq.table.slot(self.block_size, start + i) for i in range(count)]

    def commit(self, seq, num_written: int) -> None:
        """Account K/V written by a step and publish blocks that just filled
        (block_manager.py:98-120)."""
        table = seq.table
        before = table.num_filled
        table.num_filled += num_written
        self.live_tokens += num_written
        if self.live_tokens > self.peak_live_tokens:
            self.peak_live_tokens = self.live_tokens
        if not self.prefix_caching:
            return
        bs = self.block_size
        first = before // bs
        last = table.num_filled // bs
        if first >= last:
            return
        toks = seq.token_ids
        prev = self._hash_upto(seq, first)
        for i in range(first, last):
            chunk = tuple(toks[i * bs:(i + 1) * bs])
            if len(chunk) < bs:
                break
            h = hash_block(prev, chunk)
            self.allocator.mark_full(table.block_ids[i], h)
            prev = h

    def _hash_upto(self, seq, block_idx: int) -> Optional[str]:
        if block_idx == 0:
            return None
        return self.allocator.blocks[seq.table.block_ids[block_idx - 1]].content_hash

    def free(self, seq) -> None:
        for bid in seq.table.block_ids:
            self.allocator.free(bid)
        self.live_tokens -= seq.table.num_filled
        seq.table = BlockTable()

    def fork(self, parent, child) -> None:
        """Share the parent's blocks with a child (block_manager.py:133-137)."""
        child.table = BlockTable(list(parent.table.block_ids), parent.table.num_filled)
        for bid in child.table.block_ids:
            self.allocator.fork(bid)

    @property
    def usage(self) -> float:
        return 1.0 - self.allocator.num_free / self.allocator.num_blocks

    def stats(self) -> dict:
        d = self.allocator.stats()
        reserved = self.peak_blocks * self.block_size
        d.update(
            peak_blocks=self.peak_blocks,
            peak_live_tokens=self.peak_live_tokens,
            slot_utilization=(self.peak_live_tokens / reserved) if reserved else 0.0,
        )
        return d

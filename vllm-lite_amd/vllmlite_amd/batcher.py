"""Continuous batching: which requests run in the next forward pass, with how
many tokens, and which K/V blocks they write.

One `Batcher` owns the waiting queue, the running list and the block pool.
`schedule()` returns a `StepBatch`, the object a model runner's `execute`
takes: `scheduled` items (`seq`, `num_tokens`, `is_prefill`, `start_pos`) in
schedule order, `cow` (src, dst) block pairs to copy before any K/V write and
`preempted` request ids (vllmlite/scheduler.py:23-49 names these fields; a
runner reads nothing else).

The policy is the reference's (vllmlite/scheduler.py:81-164,
vllmlite/block_manager.py:26-137); the published step counts and the
reference-written streams pin it:

  * running requests first, in order, each asking for min(uncomputed tokens,
    remaining budget); a request with draft tokens that cannot push all of
    them trims them rather than splitting the guess across steps;
  * a running request that does not fit preempts the newest not-yet-scheduled
    running requests, then itself; alone in the cache and still not fitting it
    is retired with reason "cache_full";
  * waiting requests are admitted in order while budget and sequence slots
    last, first reusing any published blocks of their prompt prefix (whole
    blocks, leaving at least one prompt token to compute); a request that does
    not fit above the watermark stops admission, or is retired if the engine is
    idle and it could never fit;
  * growing a request first gives it a private copy of a shared partially
    filled block it is about to write (a copy-on-write pair), then appends
    fresh blocks; whether a request fits counts blocks from its filled tokens
    (blocks held past them after rejected drafts still count as needed);
  * preemption drops the request's K/V and puts it back at the head of the
    queue for recompute.
"""

from __future__ import annotations

from collections import deque
from typing import Deque, List, Tuple

from .kvpool import BlockList, BlockPool, chain_digest
from .request import Request, Status


class ScheduledItem:
    __slots__ = ("seq", "num_tokens", "is_prefill")

    def __init__(self, seq: Request, num_tokens: int, is_prefill: bool):
        self.seq = seq
        self.num_tokens = num_tokens
        self.is_prefill = is_prefill

    @property
    def start_pos(self) -> int:
        return self.seq.num_computed


class StepBatch:
    __slots__ = ("scheduled", "cow", "preempted")

    def __init__(self):
        self.scheduled: List[ScheduledItem] = []
        self.cow: List[Tuple[int, int]] = []
        self.preempted: List[str] = []

    @property
    def is_empty(self) -> bool:
        return not self.scheduled

    @property
    def num_batched_tokens(self) -> int:
        return sum(i.num_tokens for i in self.scheduled)

    @property
    def num_prefill_tokens(self) -> int:
        return sum(i.num_tokens for i in self.scheduled if i.is_prefill)


class Batcher:
    def __init__(self, sched_cfg, cache_cfg):
        self.cfg = sched_cfg
        self.bs = cache_cfg.block_size
        self.pool = BlockPool(cache_cfg.num_blocks, cache_cfg.block_size,
                              cache_cfg.enable_prefix_caching)
        self.waiting: Deque[Request] = deque()
        self.running: List[Request] = []
        self.finished: Deque[Request] = deque(maxlen=2048)
        self.reports: List[Request] = []
        self.watermark = int(sched_cfg.watermark * cache_cfg.num_blocks)
        self.preemptions = 0
        self.peak_blocks = 0
        self.live_tokens = 0
        self.peak_live_tokens = 0

    # -------------------------------------------------------------- requests --
    def add(self, req: Request) -> None:
        if len(self.waiting) >= self.cfg.max_waiting:
            raise RuntimeError("queue is full")
        self.waiting.append(req)

    def abort(self, request_id: str) -> bool:
        for q in (self.running, self.waiting):
            for req in q:
                if req.request_id == request_id:
                    q.remove(req)
                    self._retire(req, Status.ABORTED, "abort")
                    return True
        return False

    @property
    def has_work(self) -> bool:
        return bool(self.waiting or self.running)

    def drain_reports(self) -> List[Request]:
        out, self.reports = self.reports, []
        return out

    def finish(self, req: Request) -> None:
        """A request the engine stopped: off the running list, blocks freed."""
        if req in self.running:
            self.running.remove(req)
        self._drop_kv(req)
        self.finished.append(req)

    # ----------------------------------------------------------------- blocks --
    def _fits(self, req: Request, n: int, reserve: int = 0) -> bool:
        bs, filled = self.bs, req.table.num_filled
        need = (filled + n + bs - 1) // bs - (filled + bs - 1) // bs
        return self.pool.num_free >= need + reserve

    def _reuse_prefix(self, req: Request) -> None:
        """Take the published blocks matching the prompt's leading full blocks."""
        if not self.pool.prefix_caching or req.table.block_ids:
            return
        bs, ids, blocks = self.bs, req.ids, req.table.block_ids
        d = None
        for i in range((req.n_prompt - 1) // bs):
            d = chain_digest(d, ids[i * bs:(i + 1) * bs])
            b = self.pool.lookup(d)
            if b is None:
                break
            blocks.append(b)
        reused = len(blocks) * bs
        req.table.num_filled = req.num_computed = req.cached_prefix_tokens = reused

    def _grow(self, req: Request, n: int) -> List[Tuple[int, int]]:
        pool, bs, t = self.pool, self.bs, req.table
        blocks = t.block_ids
        cows = []
        if t.num_filled % bs:
            i = t.num_filled // bs
            if i < len(blocks) and pool.is_shared(blocks[i]):
                fresh = pool.allocate()
                cows.append((blocks[i], fresh))
                pool.release(blocks[i])
                blocks[i] = fresh
        while len(blocks) * bs < t.num_filled + n:
            blocks.append(pool.allocate())
        used = pool.num_blocks - pool.num_free
        if used > self.peak_blocks:
            self.peak_blocks = used
        return cows

    def commit(self, req: Request, n: int) -> None:
        """n more tokens of req have K/V in the cache; publish the blocks
        that just filled (their digests chain from the previous block's)."""
        t, bs = req.table, self.bs
        before = t.num_filled
        t.num_filled = before + n
        self.live_tokens += n
        if self.live_tokens > self.peak_live_tokens:
            self.peak_live_tokens = self.live_tokens
        pool = self.pool
        if not pool.prefix_caching:
            return
        first, last = before // bs, t.num_filled // bs
        if first == last:
            return
        ids, blocks = req.ids, t.block_ids
        d = pool.digest[blocks[first - 1]] if first else None
        for i in range(first, last):
            chunk = ids[i * bs:(i + 1) * bs]
            if len(chunk) < bs:
                break
            d = chain_digest(d, chunk)
            pool.publish(blocks[i], d)

    def fork(self, parent: Request, child: Request) -> None:
        """child shares every block of parent, partial tail included."""
        child.table = BlockList(list(parent.table.block_ids), parent.table.num_filled)
        for b in child.table.block_ids:
            self.pool.share(b)
        self.live_tokens += child.table.num_filled

    def _drop_kv(self, req: Request) -> None:
        for b in req.table.block_ids:
            self.pool.release(b)
        self.live_tokens -= req.table.num_filled
        req.table = BlockList()

    def _preempt(self, req: Request, out: StepBatch) -> None:
        self._drop_kv(req)
        req.restart()
        self.waiting.appendleft(req)
        out.preempted.append(req.request_id)
        self.preemptions += 1

    def _retire(self, req: Request, status: Status, reason: str) -> None:
        self._drop_kv(req)
        req.finish(status, reason)
        self.finished.append(req)
        self.reports.append(req)

    # --------------------------------------------------------------- schedule --
    def schedule(self) -> StepBatch:
        out = StepBatch()
        budget, slots = self.cfg.max_batched_tokens, self.cfg.max_seqs
        pending = deque(self.running)
        kept: List[Request] = []
        while pending:
            req = pending.popleft()
            if budget <= 0 or slots <= 0:
                kept.append(req)
                continue
            left = req.num_uncomputed
            n = min(left, budget)
            if req.n_draft and n < left:
                req.trim_drafts(n - 1)
                n = req.num_uncomputed
            while pending and not self._fits(req, n):
                self._preempt(pending.pop(), out)
            if not self._fits(req, n):
                if kept or out.scheduled:
                    self._preempt(req, out)
                else:
                    self._retire(req, Status.FINISHED_LENGTH, "cache_full")
                continue
            out.cow += self._grow(req, n)
            out.scheduled.append(ScheduledItem(req, n, req.num_uncomputed > 1))
            kept.append(req)
            budget -= n
            slots -= 1
        self.running = kept

        while self.waiting and budget > 0 and slots > 0:
            req = self.waiting[0]
            if req.num_computed == 0 and not req.table.block_ids:
                self._reuse_prefix(req)
            n = req.num_uncomputed
            if self.cfg.chunked_prefill:
                n = min(n, budget)
            elif n > budget:
                break
            if not self._fits(req, n, self.watermark):
                if not self.running and not out.scheduled and not self._fits(req, n):
                    self.waiting.popleft()
                    self._retire(req, Status.FINISHED_LENGTH, "cache_full")
                    continue
                break
            self.waiting.popleft()
            out.cow += self._grow(req, n)
            out.scheduled.append(ScheduledItem(req, n, True))
            req.status = Status.RUNNING
            self.running.append(req)
            budget -= n
            slots -= 1
        return out

    # ------------------------------------------------------------------ stats --
    def stats(self) -> dict:
        d = self.pool.stats()
        reserved = self.peak_blocks * self.bs
        d.update(peak_blocks=self.peak_blocks, peak_live_tokens=self.peak_live_tokens,
                 slot_utilization=(self.peak_live_tokens / reserved) if reserved else 0.0,
                 running=len(self.running), waiting=len(self.waiting),
                 preemptions=self.preemptions)
        return d

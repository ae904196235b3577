"""Continuous-batching scheduler with chunked prefill, recompute preemption and
prefix reuse. Behaviour follows vllmlite/scheduler.py:22-199: running
sequences are scheduled first in their running order, then waiting ones are
admitted under the remaining token budget. The order of `SchedulerOutput.
scheduled` is the order of the flattened ragged batch the kernels see.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
from typing import Deque, List, Tuple

from .block_manager import BlockManager
from .config import CacheConfig, SchedulerConfig
from .sequence import Sequence, Status


@dataclass
class ScheduledSeq:
    seq: Sequence
    num_tokens: int
    is_prefill: bool

    @property
    def start_pos(self) -> int:
        return self.seq.num_computed


@dataclass
class SchedulerOutput:
    scheduled: List[ScheduledSeq] = field(default_factory=list)
    cow: List[Tuple[int, int]] = field(default_factory=list)
    preempted: List[str] = field(default_factory=list)

    @property
    def num_batched_tokens(self) -> int:
        return sum(s.num_tokens for s in self.scheduled)

    @property
    def num_prefill_tokens(self) -> int:
        return sum(s.num_tokens for s in self.scheduled if s.is_prefill)

    @property
    def is_empty(self) -> bool:
        return not self.scheduled


class Scheduler:
    def __init__(self, sched_cfg: SchedulerConfig, cache_cfg: CacheConfig):
        self.cfg = sched_cfg
        self.blocks = BlockManager(cache_cfg)
        self.waiting: Deque[Sequence] = deque()
        self.running: List[Sequence] = []
        self.finished: Deque[Sequence] = deque(maxlen=2048)
        self.pending_reports: List[Sequence] = []
        self.watermark_blocks = int(sched_cfg.watermark * cache_cfg.num_blocks)
        self.total_preemptions = 0

    def add(self, seq: Sequence) -> None:
        if len(self.waiting) >= self.cfg.max_waiting:
            raise RuntimeError("queue is full")
        self.waiting.append(seq)

    def abort(self, request_id: str) -> bool:
        for pool in (self.running, self.waiting):
            for seq in list(pool):
                if seq.request_id == request_id:
                    pool.remove(seq)
                    self._retire(seq, Status.ABORTED, "abort")
                    return True
        return False

    @property
    def has_work(self) -> bool:
        return bool(self.waiting or self.running)

    def drain_reports(self) -> List[Sequence]:
        out, self.pending_reports = self.pending_reports, []
        return out

    def schedule(self) -> SchedulerOutput:
        out = SchedulerOutput()
        budget = self.cfg.max_batched_tokens
        slots = self.cfg.max_seqs
        blocks = self.blocks

        # 1. sequences that already hold blocks (scheduler.py:98-134)
        queue = deque(self.running)
        keep: List[Sequence] = []
        while queue:
            seq = queue.popleft()
            if budget <= 0 or slots <= 0:
                keep.append(seq)
                continue
            want = min(seq.num_uncomputed, budget)
            if seq.draft_token_ids and want < seq.num_uncomputed:
                # never split a speculation across steps: shorten the guess
                seq.trim_drafts(want - 1)
                want = seq.num_uncomputed
            # newest unscheduled sequences give their blocks up first
            while queue and not blocks.can_allocate(seq, want):
                self._preempt(queue.pop(), out)
            if not blocks.can_allocate(seq, want):
                if not keep and out.is_empty:
                    self._retire(seq, Status.FINISHED_LENGTH, "cache_full")
                else:
                    self._preempt(seq, out)
                continue
            out.cow += blocks.append_slots(seq, want)
            out.scheduled.append(ScheduledSeq(seq, want, seq.num_uncomputed > 1))
            keep.append(seq)
            budget -= want
            slots -= 1
        self.running = keep

        # 2. admissions under the remaining budget (scheduler.py:137-164)
        while self.waiting and budget > 0 and slots > 0:
            seq = self.waiting[0]
            if seq.num_computed == 0 and not seq.table.block_ids:
                blocks.reuse_prefix(seq)
            want = seq.num_uncomputed
            if self.cfg.chunked_prefill:
                want = min(want, budget)
            elif want > budget:
                break
            if not blocks.can_allocate(seq, want, self.watermark_blocks):
                if not self.running and out.is_empty and not blocks.can_allocate(seq, want):
                    # longer than the whole cache: retire instead of spinning
                    self.waiting.popleft()
                    self._retire(seq, Status.FINISHED_LENGTH, "cache_full")
                    continue
                break
            self.waiting.popleft()
            out.cow += blocks.append_slots(seq, want)
            out.scheduled.append(ScheduledSeq(seq, want, True))
            seq.status = Status.RUNNING
            self.running.append(seq)
            budget -= want
            slots -= 1
        return out

    def _preempt(self, seq: Sequence, out: SchedulerOutput) -> None:
        self.blocks.free(seq)
        seq.reset_for_recompute()
        self.waiting.appendleft(seq)
        out.preempted.append(seq.request_id)
        self.total_preemptions += 1

    def _retire(self, seq: Sequence, status: Status, reason: str) -> None:
        self.blocks.free(seq)
        seq.finish(status, reason)
        self.finished.append(seq)
        self.pending_reports.append(seq)

    def finish(self, seq: Sequence) -> None:
        if seq in self.running:
            self.running.remove(seq)
        self.blocks.free(seq)
        self.finished.append(seq)

    def stats(self) -> dict:
        d = self.blocks.stats()
        d.update(running=len(self.running), waiting=len(self.waiting),
                 preemptions=self.total_preemptions)
        return d

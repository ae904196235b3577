"""Request state: status, sampling parameters, the sequence and its output.

Behaviour follows vllmlite/sequence.py:10-149. `token_ids` is prompt, then
outputs, then unverified drafts (sequence.py:69-71); the runner reads it to
find the tokens a step pushes through the model.
"""

from __future__ import annotations

import enum
import time
from dataclasses import dataclass, field
from typing import List, Optional

from .block import BlockTable


class Status(enum.Enum):
    WAITING = "waiting"
    RUNNING = "running"
    PREEMPTED = "preempted"
    FINISHED_STOP = "finished_stop"
    FINISHED_LENGTH = "finished_length"
    ABORTED = "aborted"

    @property
    def finished(self) -> bool:
        return self in _FINISHED


_FINISHED = frozenset((Status.FINISHED_STOP, Status.FINISHED_LENGTH, Status.ABORTED))


@dataclass
class SamplingParams:
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = 0
    max_tokens: int = 64
    min_tokens: int = 0
    stop: List[str] = field(default_factory=list)
    stop_token_ids: List[int] = field(default_factory=list)
    repetition_penalty: float = 1.0
    seed: Optional[int] = None
    ignore_eos: bool = False

    def __post_init__(self):
        # sequence.py:36-42
        if self.temperature < 0:
            raise ValueError("temperature must be >= 0")
        if not 0 < self.top_p <= 1:
            raise ValueError("top_p must be in (0, 1]")
        if self.max_tokens < 1:
            raise ValueError("max_tokens must be >= 1")

    @property
    def greedy(self) -> bool:
        return self.temperature == 0.0


@dataclass
class Sequence:
    request_id: str
    prompt_token_ids: List[int]
    params: SamplingParams
    status: Status = Status.WAITING
    output_token_ids: List[int] = field(default_factory=list)
    draft_token_ids: List[int] = field(default_factory=list)
    table: BlockTable = field(default_factory=BlockTable)
    # tokens of this sequence whose K/V is already in the cache
    num_computed: int = 0
    arrival: float = field(default_factory=time.perf_counter)
    first_token_at: Optional[float] = None
    finished_at: Optional[float] = None
    preempt_count: int = 0
    cached_prefix_tokens: int = 0
    stop_reason: Optional[str] = None

    @property
    def token_ids(self) -> List[int]:
        return self.prompt_token_ids + self.output_token_ids + self.draft_token_ids

    def token_slice(self, start: int, stop: int) -> List[int]:
        """token_ids[start:stop] without building the whole concatenation."""
        p = self.prompt_token_ids
        np_ = len(p)
        if stop <= np_:
            return p[start:stop]
        return self.token_ids[start:stop]

    @property
    def num_tokens(self) -> int:
        return len(self.prompt_token_ids) + len(self.output_token_ids) + len(self.draft_token_ids)

    def trim_drafts(self, keep: int) -> None:
        del self.draft_token_ids[keep:]

    @property
    def num_prompt_tokens(self) -> int:
        return len(self.prompt_token_ids)

    @property
    def is_prefill(self) -> bool:
        return self.num_uncomputed > 1

    @property
    def num_uncomputed(self) -> int:
        return self.num_tokens - self.num_computed

    def append_token(self, token_id: int) -> None:
        self.output_token_ids.append(token_id)
        if self.first_token_at is None:
            self.first_token_at = time.perf_counter()

    def reset_for_recompute(self) -> None:
        """Preemption by recompute (sequence.py:101-108): the K/V goes, the tokens stay."""
        self.draft_token_ids.clear()
        self.num_computed = 0
        self.cached_prefix_tokens = 0
        self.table = BlockTable()
        self.preempt_count += 1
        self.status = Status.PREEMPTED

    def finish(self, status: Status, reason: Optional[str] = None) -> None:
        self.status = status
        self.stop_reason = reason
        self.finished_at = time.perf_counter()

    @property
    def ttft(self) -> Optional[float]:
        return None if self.first_token_at is None else self.first_token_at - self.arrival

    @property
    def e2e(self) -> Optional[float]:
        return None if self.finished_at is None else self.finished_at - self.arrival

    @property
    def tpot(self) -> Optional[float]:
        if self.first_token_at is None or self.finished_at is None:
            return None
        n = len(self.output_token_ids) - 1
        if n <= 0:
            return None
        return (self.finished_at - self.first_token_at) / n


@dataclass
class RequestOutput:
    request_id: str
    token_ids: List[int]
    new_token_ids: List[int]
    text_delta: str
    finished: bool
    finish_reason: Optional[str] = None
    num_prompt_tokens: int = 0
    num_output_tokens: int = 0
    cached_prefix_tokens: int = 0

"""Requests as the engine tracks them.

`SamplingParams` and `RequestOutput` keep the reference's field names,
defaults and validation (vllmlite/sequence.py:22-42, 138-149): they are what a
caller of the reference constructs and reads. `Request` is this package's
record of one sequence. Its token ids live in ONE list, prompt then outputs
then the current draft tokens, so the runner's slice
`token_ids[start:start + n]` (vllmlite/runner.py:74-76) is a single list
slice (`token_slice`), and the attributes the runner reads carry the
reference's names: `token_ids`, `num_computed`, `draft_token_ids`,
`table.block_ids`, `request_id`.
"""

from __future__ import annotations

import enum
import time
from dataclasses import dataclass, field
from typing import List, Optional

from .kvpool import BlockList


class Status(enum.Enum):
    WAITING = "waiting"
    RUNNING = "running"
    PREEMPTED = "preempted"
    FINISHED_STOP = "finished_stop"
    FINISHED_LENGTH = "finished_length"
    ABORTED = "aborted"

    @property
    def finished(self) -> bool:
        return self._finished


# per member, as plain attributes: the engine asks these of every running
# request every step, and an Enum member's hash is a Python-level call
_REASONS = {Status.FINISHED_STOP: "stop", Status.FINISHED_LENGTH: "length",
            Status.ABORTED: "abort"}
for _s in Status:
    _s._finished = _s in _REASONS
    _s._reason = _REASONS.get(_s)
del _s


def finish_reason(status: Status) -> Optional[str]:
    return status._reason


@dataclass
class SamplingParams:
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = 0  # 0 disables
    max_tokens: int = 64
    min_tokens: int = 0
    stop: List[str] = field(default_factory=list)
    stop_token_ids: List[int] = field(default_factory=list)
    repetition_penalty: float = 1.0
    seed: Optional[int] = None
    ignore_eos: bool = False

    def __post_init__(self):
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


class Request:
    __slots__ = ("request_id", "params", "status", "ids", "n_prompt", "n_draft", "table",
                 "num_computed", "arrival", "first_token_at", "finished_at", "preempt_count",
                 "cached_prefix_tokens", "stop_reason", "text", "decoder", "rng")

    def __init__(self, request_id: str, prompt_token_ids: List[int], params: SamplingParams):
        self.request_id = request_id
        self.params = params
        self.status = Status.WAITING
        self.ids: List[int] = list(prompt_token_ids)
        self.n_prompt = len(self.ids)
        self.n_draft = 0
        self.table = BlockList()
        self.num_computed = 0
        self.arrival = time.perf_counter()
        self.first_token_at: Optional[float] = None
        self.finished_at: Optional[float] = None
        self.preempt_count = 0
        self.cached_prefix_tokens = 0
        self.stop_reason: Optional[str] = None
        self.text = ""
        self.decoder = None
        self.rng = None

    # ----------------------------------------------------- runner-facing view --
    @property
    def token_ids(self) -> List[int]:
        return list(self.ids)

    def token_slice(self, start: int, stop: int) -> List[int]:
        return self.ids[start:stop]

    @property
    def draft_token_ids(self) -> List[int]:
        return self.ids[len(self.ids) - self.n_draft:] if self.n_draft else []

    # ---------------------------------------------------------------- counts --
    @property
    def num_tokens(self) -> int:
        return len(self.ids)

    @property
    def num_uncomputed(self) -> int:
        return len(self.ids) - self.num_computed

    @property
    def num_output(self) -> int:
        return len(self.ids) - self.n_prompt - self.n_draft

    @property
    def num_prompt_tokens(self) -> int:
        return self.n_prompt

    @property
    def prompt_token_ids(self) -> List[int]:
        return self.ids[:self.n_prompt]

    @property
    def output_token_ids(self) -> List[int]:
        return self.ids[self.n_prompt:len(self.ids) - self.n_draft]

    def context_ids(self) -> List[int]:
        """Prompt and outputs, without drafts."""
        return self.ids[:len(self.ids) - self.n_draft] if self.n_draft else self.ids

    # --------------------------------------------------------------- updates --
    def set_drafts(self, drafts: List[int]) -> None:
        self.clear_drafts()
        self.ids.extend(drafts)
        self.n_draft = len(drafts)

    def trim_drafts(self, keep: int) -> None:
        if keep < self.n_draft:
            del self.ids[len(self.ids) - self.n_draft + keep:]
            self.n_draft = keep

    def clear_drafts(self) -> None:
        if self.n_draft:
            del self.ids[len(self.ids) - self.n_draft:]
            self.n_draft = 0

    def append_token(self, token_id: int) -> None:
        self.ids.append(token_id)
        if self.first_token_at is None:
            self.first_token_at = time.perf_counter()

    def restart(self) -> None:
        """Preemption by recompute: the K/V is dropped, the tokens are kept."""
        self.clear_drafts()
        self.num_computed = 0
        self.cached_prefix_tokens = 0
        self.table = BlockList()
        self.preempt_count += 1
        self.status = Status.PREEMPTED

    def finish(self, status: Status, reason: Optional[str] = None) -> None:
        self.status = status
        self.stop_reason = reason
        self.finished_at = time.perf_counter()

    # ---------------------------------------------------------------- timing --
    @property
    def ttft(self) -> Optional[float]:
        return None if self.first_token_at is None else self.first_token_at - self.arrival

    @property
    def e2e(self) -> Optional[float]:
        return None if self.finished_at is None else self.finished_at - self.arrival

    @property
    def tpot(self) -> Optional[float]:
        n = self.num_output - 1
        if self.first_token_at is None or self.finished_at is None or n <= 0:
            return None
        return (self.finished_at - self.first_token_at) / n

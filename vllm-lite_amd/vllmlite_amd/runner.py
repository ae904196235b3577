"""The model-runner boundary.

`ModelRunner` is the reference's plug-in interface (vllmlite/runner.py:19-32):
`execute(SchedulerOutput) -> (logits, rows)` where logits is a host float32
array [R, vocab] and rows[i] = (first_row, count) for the i'th scheduled
sequence. The GPU implementation is `hip_runner.HipRunner`, which flattens the
batch itself (`hip_runner.flatten_scheduled`).
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import List, Tuple

import numpy as np


class ModelRunner(ABC):
    @abstractmethod
    def execute(self, out) -> Tuple[np.ndarray, List[Tuple[int, int]]]:
        """Returns (logits, rows); rows[i] is (first_row, count), count being 1
        for plain decoding and 1 + num_drafts when speculating."""

    @property
    @abstractmethod
    def vocab_size(self) -> int: ...


def make_runner(cfg) -> ModelRunner:
    if cfg.backend == "hip":
        from .hip_runner import HipRunner
        return HipRunner(cfg.model, cfg.cache)
    raise ValueError(
        f"backend {cfg.backend!r} is not provided by this package; "
        "use backend='hip' or pass runner= to LLMEngine")

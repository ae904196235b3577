"""The model-runner boundary and the ragged-batch flattening shared by runners.

`ModelRunner` is the reference's plug-in interface (vllmlite/runner.py:19-32):
`execute(SchedulerOutput) -> (logits, rows)` where logits is a host float32
array [R, vocab] and rows[i] = (first_row, count) for the i'th scheduled
sequence. The GPU implementation is `hip_runner.HipRunner`.

`flatten_batch` restates the flattening of runner.py:62-100 as int32 arrays
in the layout the kernels read (one row per scheduled sequence, in schedule
order):

    query_start_loc[S+1]   prefix sum of tokens pushed this step
    seq_lens[S]            context after this step's writes (start + n)
    block_tables[S, W]     physical block ids, padded with 0
    slot_mapping[T]        flat cache slot of every new token
    positions[T]           absolute position of every new token
    token_ids[T]
    logits_idx[R]          token rows whose logits the engine reads
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass
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


@dataclass
class FlatBatch:
    token_ids: np.ndarray
    positions: np.ndarray
    query_start_loc: np.ndarray
    seq_lens: np.ndarray
    block_tables: np.ndarray
    slot_mapping: np.ndarray
    logits_idx: np.ndarray
    rows: List[Tuple[int, int]]

    @property
    def num_tokens(self) -> int:
        return int(self.token_ids.shape[0])

    @property
    def num_seqs(self) -> int:
        return int(self.seq_lens.shape[0])


def flatten_batch(out, block_size: int, min_table_width: int = 1) -> FlatBatch:
    """SchedulerOutput -> FlatBatch. Sequence i contributes tokens
    token_ids[start:start+n] at positions start..start+n-1 with start =
    seq.num_computed (scheduler.py:28-30, runner.py:72-80); its slots are
    block_ids[p // bs] * bs + p % bs (block.py:154-156); it asks for
    min(1 + len(drafts), n) logit rows, the last ones of its tokens
    (runner.py:86-90)."""
    sched = out.scheduled
    S = len(sched)
    ns = np.empty(S, dtype=np.int64)
    starts = np.empty(S, dtype=np.int64)
    width = min_table_width
    toks: List[int] = []
    counts = np.empty(S, dtype=np.int64)
    for i, item in enumerate(sched):
        seq = item.seq
        start = seq.num_computed
        n = item.num_tokens
        starts[i] = start
        ns[i] = n
        toks += seq.token_slice(start, start + n)
        nd = len(seq.draft_token_ids)
        counts[i] = min(1 + nd, n)
        nb = len(seq.table.block_ids)
        if nb > width:
            width = nb
    tables = np.zeros((S, width), dtype=np.int32)
    for i, item in enumerate(sched):
        ids = item.seq.table.block_ids
        tables[i, :len(ids)] = ids
    qsl = np.zeros(S + 1, dtype=np.int64)
    np.cumsum(ns, out=qsl[1:])
    T = int(qsl[-1])
    seq_of_tok = np.repeat(np.arange(S), ns)
    positions = np.arange(T, dtype=np.int64) - qsl[:-1][seq_of_tok] + starts[seq_of_tok]
    blk = tables[seq_of_tok, positions // block_size].astype(np.int64)
    slots = blk * block_size + positions % block_size
    # logits rows: the last `count` tokens of every sequence
    ends = qsl[1:]
    rsl = np.zeros(S + 1, dtype=np.int64)
    np.cumsum(counts, out=rsl[1:])
    R = int(rsl[-1])
    seq_of_row = np.repeat(np.arange(S), counts)
    logits_idx = ends[seq_of_row] - counts[seq_of_row] + (np.arange(R) - rsl[:-1][seq_of_row])
    rows = [(int(rsl[i]), int(counts[i])) for i in range(S)]
    return FlatBatch(
        token_ids=np.asarray(toks, dtype=np.int32),
        positions=positions.astype(np.int32),
        query_start_loc=qsl.astype(np.int32),
        seq_lens=(starts + ns).astype(np.int32),
        block_tables=tables,
        slot_mapping=slots.astype(np.int32),
        logits_idx=logits_idx.astype(np.int32),
        rows=rows,
    )


def make_runner(cfg) -> ModelRunner:
    if cfg.backend == "hip":
        from .hip_runner import HipRunner
        return HipRunner(cfg.model, cfg.cache)
    raise ValueError(
        f"backend {cfg.backend!r} is not provided by this package; "
        "use backend='hip' or pass runner= to LLMEngine")

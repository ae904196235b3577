"""HipRunner's batch flattening under objects shaped exactly like the
reference's own types, on the CPU.

The reference runner reads `item.start_pos`, `item.num_tokens`,
`seq.token_ids[start:start + n]`, `seq.draft_token_ids` and
`seq.table.block_ids` (vllmlite/runner.py:72-90). The classes below carry the
attribute sets of the reference's `BlockTable` (vllmlite/block.py:120-156),
`Sequence` (vllmlite/sequence.py:49-94), `ScheduledSeq` and `SchedulerOutput`
(vllmlite/scheduler.py:23-49) and nothing else (`__slots__`), so a runner that
needs any other member fails here. The expected flattening is the oracle
runner's (oracle/runner.py, restating runner.py:62-100).
"""

import numpy as np
import pytest

pytest.importorskip("torch")

from vllmlite_amd.config import CacheConfig, ModelConfig  # noqa: E402
from vllmlite_amd.hip_runner import flatten_scheduled, fused_rows_supported  # noqa: E402
from oracle.runner import NumpyRunner  # noqa: E402


class RefBlockTable:
    __slots__ = ("block_ids", "num_filled")

    def __init__(self, block_ids=None, num_filled=0):
        self.block_ids = list(block_ids or [])
        self.num_filled = num_filled

    def slot(self, block_size, pos):
        return self.block_ids[pos // block_size] * block_size + pos % block_size


class RefSequence:
    __slots__ = ("request_id", "prompt_token_ids", "params", "status", "output_token_ids",
                 "draft_token_ids", "table", "num_computed", "arrival", "first_token_at",
                 "finished_at", "preempt_count", "cached_prefix_tokens", "stop_reason")

    def __init__(self, rid, prompt, output, drafts, blocks, num_computed):
        self.request_id = rid
        self.prompt_token_ids = list(prompt)
        self.params = None
        self.status = None
        self.output_token_ids = list(output)
        self.draft_token_ids = list(drafts)
        self.table = RefBlockTable(blocks, num_computed)
        self.num_computed = num_computed
        self.arrival = self.first_token_at = self.finished_at = None
        self.preempt_count = self.cached_prefix_tokens = 0
        self.stop_reason = None

    @property
    def token_ids(self):
        return self.prompt_token_ids + self.output_token_ids + self.draft_token_ids

    @property
    def num_tokens(self):
        return len(self.prompt_token_ids) + len(self.output_token_ids) + len(self.draft_token_ids)

    @property
    def num_uncomputed(self):
        return self.num_tokens - self.num_computed


class RefScheduledSeq:
    __slots__ = ("seq", "num_tokens", "is_prefill")

    def __init__(self, seq, num_tokens, is_prefill):
        self.seq, self.num_tokens, self.is_prefill = seq, num_tokens, is_prefill

    @property
    def start_pos(self):
        return self.seq.num_computed


class RefSchedulerOutput:
    __slots__ = ("scheduled", "cow", "preempted")

    def __init__(self, scheduled, cow=()):
        self.scheduled, self.cow, self.preempted = list(scheduled), list(cow), []


def _batch(rng, bs):
    """A prefill chunk, a plain decode, a speculating decode (3 drafts), a
    recompute after preemption and a one-token prompt, over scattered blocks."""
    perm = [int(x) for x in rng.permutation(64)]
    specs = [  # (prompt, output, drafts, num_computed, tokens this step)
        (40, 0, 0, 16, 24),
        (21, 7, 0, 27, 1),
        (30, 5, 3, 34, 4),
        (12, 9, 0, 0, 21),
        (1, 0, 0, 0, 1),
    ]
    items, off = [], 0
    for i, (p, o, d, done, n) in enumerate(specs):
        nb = -(-(done + n) // bs)
        seq = RefSequence(f"s{i}", rng.integers(0, 261, p), rng.integers(0, 261, o),
                          rng.integers(0, 261, d), perm[off:off + nb], done)
        off += nb
        items.append(RefScheduledSeq(seq, n, n > 1))
    return RefSchedulerOutput(items)


@pytest.mark.parametrize("bs", [4, 16])
def test_flatten_reads_only_reference_fields(bs):
    out = _batch(np.random.default_rng(bs), bs)
    f = flatten_scheduled(out, bs, 512)
    mc = ModelConfig(n_layers=1, n_heads=4, n_kv_heads=2, d_model=32, d_ff=32, max_seq_len=512)
    ref = NumpyRunner(mc, CacheConfig(block_size=bs, num_blocks=64))
    _, rows = ref.execute(out)
    token_ids, positions, seq_meta, want = ref.last_batch
    assert f.toks == [int(t) for t in token_ids]
    assert f.pos == list(positions)
    assert f.lidx == list(want)
    assert f.rows == rows
    assert f.T == len(token_ids) and f.R == len(want) and f.S == len(out.scheduled)
    for i, (offset, n, write_slots, read_slots) in enumerate(seq_meta):
        assert f.qsl[i] == offset and f.qsl[i + 1] == offset + n
        assert f.slots[offset:offset + n] == [int(x) for x in write_slots]
        assert f.lens[i] == len(read_slots)
        blocks = f.tables[i]
        rebuilt = [blocks[p // bs] * bs + p % bs for p in range(len(read_slots))]
        assert rebuilt == [int(x) for x in read_slots]


def test_flatten_rejects_missing_blocks_and_positions_past_max_len():
    rng = np.random.default_rng(0)
    out = _batch(rng, 16)
    out.scheduled[0].seq.table.block_ids.pop()
    with pytest.raises(ValueError):
        flatten_scheduled(out, 16, 512)
    with pytest.raises(IndexError):
        flatten_scheduled(_batch(rng, 16), 16, 30)


def test_fused_row_kernels_only_for_supported_shapes():
    """d_model 72 (4 heads of 18) is a valid ModelConfig (vllmlite/config.py:20-24)
    but not a multiple of 16: such models take the GEMM path and keep no tiled
    weight copies."""
    assert not fused_rows_supported(ModelConfig(n_heads=4, n_kv_heads=2, d_model=72, d_ff=128))
    assert not fused_rows_supported(ModelConfig(d_model=512, d_ff=2048))
    assert fused_rows_supported(ModelConfig(n_heads=8, n_kv_heads=4, d_model=384, d_ff=1024))

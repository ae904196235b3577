"""HipRunner's host staging (RecordStager): the int32 record it writes for
every step of the published mixes, copy-on-write forks included, equals the
record built from scratch out of flatten_scheduled (runner.py:62-100's
flattening), in every buffer of the two it alternates between. No GPU."""

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path[:0] = [ROOT, os.path.join(ROOT, "vllm-lite_amd")]

from vllmlite_amd.hip_runner import RecordStager, _Shape, _bucket, flatten_scheduled  # noqa: E402


def full_record(out, bs, max_len, W, short_decode, n):
    """The record as flatten_scheduled describes it (every table row written,
    rows past a table's length zero)."""
    f = flatten_scheduled(out, bs, max_len)
    s = _Shape(_bucket(f.T, 16), _bucket(f.S, 8), _bucket(f.R, 8), W,
               f.max_q == 1 and short_decode)
    m = np.zeros(n, np.int32)
    T, S, R = f.T, f.S, f.R
    m[s.tok:s.tok + s.Tb] = f.toks + [0] * (s.Tb - T)
    m[s.pos:s.pos + s.Tb] = f.pos + [0] * (s.Tb - T)
    m[s.slot:s.slot + s.Tb] = f.slots + [-1] * (s.Tb - T)
    m[s.lidx:s.lidx + s.Rb] = f.lidx + [0] * (s.Rb - R)
    m[s.qsl:s.qsl + s.Sb + 1] = f.qsl + [T] * (s.Sb - S)
    m[s.lens:s.lens + s.Sb] = f.lens + [0] * (s.Sb - S)
    for i, ids in enumerate(f.tables):
        m[s.bt + i * W:s.bt + i * W + len(ids)] = ids
    return s, f, m


class StagingRunner:
    """A runner that stages each step with RecordStager and checks it."""

    def __init__(self, cfg):
        self.cfg = cfg
        self.bs = cfg.cache.block_size
        self.W = -(-cfg.model.max_seq_len // self.bs)
        self.n = _Shape(4096, 4096, 4096, self.W).n_ints
        self.bufs = [np.full(self.n, 12345, np.int32) for _ in range(2)]
        self.stager = RecordStager(2)
        self.k = 0
        self.steps = self.cow_steps = 0
        self.vocab_size = cfg.model.vocab_size

    def execute(self, out):
        mc = self.cfg.model
        k = self.k
        self.k ^= 1
        m = self.bufs[k]
        shape, rows, R, T, width = self.stager.stage(out, m, k, self.bs, mc.max_seq_len, self.W,
                                                     True, 4096)
        s, f, want = full_record(out, self.bs, mc.max_seq_len, self.W, True, self.n)
        assert shape is not None and (shape.Tb, shape.Sb, shape.Rb, shape.decode) == (
            s.Tb, s.Sb, s.Rb, s.decode)
        assert rows == f.rows and R == f.R and T == f.T and width == f.width
        np.testing.assert_array_equal(m[:s.bt], want[:s.bt])
        for i, ids in enumerate(f.tables):  # each row's entries up to its length
            np.testing.assert_array_equal(m[s.bt + i * s.W:s.bt + i * s.W + len(ids)], ids)
        self.steps += 1
        self.cow_steps += bool(out.cow)
        return np.zeros((R, self.vocab_size), np.float32), rows


@pytest.mark.parametrize("mix", ["mixed", "shared_prefix", "shared_prefix_forked"])
def test_stager_matches_flatten_on_the_mixes(mix):
    import bench
    from vllmlite_amd.engine import LLMEngine
    from vllmlite_amd.workload import drive_forked, mixed_lengths
    cfg = bench.mix_config(mix)
    r = StagingRunner(cfg)
    eng = LLMEngine(cfg, runner=r)
    eng.device_argmax = False
    shared, fork = bench.MIXES[mix]
    reqs = mixed_lengths(0, 48, shared)
    if fork:
        drive_forked(eng, reqs)
    else:
        for rid, ids, p in reqs:
            eng.add_request(params=p, request_id=rid, prompt_token_ids=ids)
        while eng.has_work:
            eng.step()
    assert r.steps >= 250
    if fork:
        assert r.cow_steps > 0


def test_stager_rows_follow_new_and_preempted_tables():
    """A tiny cache that preempts and re-admits requests: tables replaced at
    the same row, shrunk and regrown, every step still equal."""
    from vllmlite_amd.config import CacheConfig, EngineConfig, ModelConfig, SchedulerConfig
    from vllmlite_amd.engine import LLMEngine
    from vllmlite_amd.request import SamplingParams
    cfg = EngineConfig(model=ModelConfig(n_layers=1, d_model=64, n_heads=4, n_kv_heads=2,
                                         d_ff=128, max_seq_len=256),
                       cache=CacheConfig(block_size=4, num_blocks=24),
                       scheduler=SchedulerConfig(max_batched_tokens=64, max_seqs=4))
    r = StagingRunner(cfg)
    eng = LLMEngine(cfg, runner=r)
    eng.device_argmax = False
    rng = np.random.default_rng(5)
    for i in range(10):
        ids = rng.integers(0, 256, int(rng.integers(5, 30))).tolist()
        eng.add_request(params=SamplingParams(max_tokens=int(rng.integers(3, 25)), temperature=0,
                                              ignore_eos=True),
                        request_id=f"r{i}", prompt_token_ids=ids)
    while eng.has_work:
        eng.step()
    assert eng.batcher.preemptions > 0
    assert r.steps > 20

"""The oracle and the restated caller side against fixtures the reference
itself pins: published workload totals and step counts
(results/mixed_lengths.json:22-23,88-91; results/shared_prefix.json), seeded
weight hashes and end-to-end greedy streams written from the reference by
tests/golden/make_golden.py."""

import hashlib
import json
import os

import numpy as np
import pytest

from vllmlite_amd.config import ModelConfig
from vllmlite_amd.engine import LLMEngine
from vllmlite_amd.workload import mixed_lengths
from oracle.model import init_weights
from oracle.runner import NumpyRunner

from helpers import cfg0_config

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _load(name):
    with open(os.path.join(GOLD, name)) as f:
        return json.load(f)


def _drive(prefix_cache, shared):
    cfg = cfg0_config(prefix_cache)
    eng = LLMEngine(cfg, runner=NumpyRunner(cfg.model, cfg.cache))
    reqs = mixed_lengths(0, 48, shared)
    for rid, ids, p in reqs:
        eng.add_request(params=p, request_id=rid, prompt_token_ids=ids)
    while eng.has_work:
        eng.step()
    return eng, reqs


def test_workload_matches_published_totals():
    reqs = mixed_lengths(0, 48, 0)
    assert sum(len(r[1]) for r in reqs) == 3025
    assert sum(r[2].max_tokens for r in reqs) == 3179
    shared = mixed_lengths(0, 48, 256)
    assert sum(len(r[1]) for r in shared) == 14480
    assert sum(r[2].max_tokens for r in shared) == 3323


def test_workload_matches_golden_prompts():
    g = _load("cfg0_streams.json")
    for rid, ids, _ in mixed_lengths(0, 48, 0):
        assert ids == g["prompts"][rid]


@pytest.mark.parametrize("name,mc", [
    ("cfg0", ModelConfig(n_layers=6, n_heads=8, n_kv_heads=4, d_model=384, d_ff=1024,
                         vocab_size=261, max_seq_len=512)),
    ("small", ModelConfig(n_layers=2, n_heads=4, n_kv_heads=2, d_model=64, d_ff=128, max_seq_len=512)),
])
def test_oracle_weights_match_reference_hashes(name, mc):
    want = _load("weights_sha256.json")[name]
    w = init_weights(mc)
    for key, h in want.items():
        assert hashlib.sha256(np.ascontiguousarray(w[key]).tobytes()).hexdigest() == h, key


def test_oracle_engine_reproduces_reference_streams_and_steps():
    g = _load("cfg0_streams.json")
    eng, reqs = _drive(False, 0)
    assert eng.total_steps == g["steps"] == 260
    st = eng.stats()
    assert st["prompt_tokens"] == 3025 and st["output_tokens"] == 3179
    assert st["preemptions"] == 0 and round(st["slot_utilization"], 3) == 0.942
    for rid, _, _ in reqs:
        assert eng.seqs[rid].output_token_ids == g["streams"][rid], rid


def test_shared_prefix_step_counts():
    eng, _ = _drive(False, 256)
    st = eng.stats()
    assert (st["steps"], round(st["slot_utilization"], 3)) == (281, 0.978)
    eng, _ = _drive(True, 256)
    st = eng.stats()
    assert (st["steps"], round(st["slot_utilization"], 3), st["prefix_hit_rate"]) == (280, 0.629, 1.0)


def _cfg3(prefix_cache=True):
    from vllmlite_amd.workload import shared_prefix_config
    cfg = shared_prefix_config(prefix_cache)
    return LLMEngine(cfg, runner=NumpyRunner(cfg.model, cfg.cache))


def test_shared_prefix_mix_matches_reference_streams():
    """The published shared-prefix configuration (max_len 768, 768 blocks,
    prefix cache on): 280 steps and the reference's 3323-token streams."""
    g = _load("shared_prefix_streams.json")
    eng = _cfg3()
    reqs = mixed_lengths(0, 48, 256)
    for rid, ids, p in reqs:
        assert ids == g["prompts"][rid]
        eng.add_request(params=p, request_id=rid, prompt_token_ids=ids)
    while eng.has_work:
        eng.step()
    assert eng.total_steps == g["plain"]["steps"] == 280
    assert eng.total_output_tokens == g["plain"]["output_tokens"] == 3323
    for rid, _, _ in reqs:
        assert eng.seqs[rid].output_token_ids == g["plain"]["streams"][rid], rid


def test_forked_shared_prefix_mix_matches_reference():
    """Every request forked once after its first token (BlockManager.fork,
    vllmlite/block_manager.py:133-137): the reference's step count, copy-on-
    write pair count (one per partial shared tail) and every stream, parents
    and children."""
    from vllmlite_amd.workload import drive_forked
    g = _load("shared_prefix_streams.json")["forked"]
    eng = _cfg3()
    pairs = []
    execute = eng.runner.execute

    def counting(out):
        pairs.extend(out.cow)
        return execute(out)

    eng.runner.execute = counting
    forked, partial = drive_forked(eng, mixed_lengths(0, 48, 256))
    assert sorted(forked) == sorted(g["forked"]) and partial == g["partial_tails"]
    assert len(pairs) == g["cow_pairs"] == len(partial) == 44
    assert eng.total_steps == g["steps"]
    assert eng.total_output_tokens == g["output_tokens"]
    assert {rid: s.output_token_ids for rid, s in eng.seqs.items()} == g["streams"]

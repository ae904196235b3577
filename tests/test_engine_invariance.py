"""Greedy output must not depend on paging, chunking, batching, prefix caching
or preemption (the reference's tests/test_engine.py:57-204), here on the
restated caller side driving the NumPy oracle runner. The expected streams are
the reference's own, from tests/golden/small_streams.json."""

import json
import os

import numpy as np
import pytest

from oracle.runner import NumpyRunner
from vllmlite_amd.request import SamplingParams
from vllmlite_amd.sampling import choose

from helpers import PROMPTS, build, run

GOLD = os.path.join(os.path.dirname(__file__), "golden", "small_streams.json")


def reference():
    with open(GOLD) as f:
        g = json.load(f)
    assert g["prompts"] == PROMPTS
    return g["streams"]


def test_default_engine_matches_reference_streams():
    assert run(build(), PROMPTS, check_counts=True) == reference()


@pytest.mark.parametrize("block_size", [1, 4, 16, 64])
def test_block_size_does_not_change_output(block_size):
    assert run(build(block_size=block_size), PROMPTS) == reference()


def test_prefix_caching_does_not_change_output():
    assert run(build(prefix_cache=True), PROMPTS, check_counts=True) == reference()


@pytest.mark.parametrize("max_batched", [8, 33, 64, 4096])
def test_chunked_prefill_does_not_change_output(max_batched):
    assert run(build(max_batched=max_batched), PROMPTS) == reference()


def test_no_chunked_prefill_matches():
    assert run(build(chunked=False, max_batched=4096), PROMPTS) == reference()


@pytest.mark.parametrize("max_seqs", [1, 2, 3, 8])
def test_batch_composition_does_not_change_output(max_seqs):
    assert run(build(max_seqs=max_seqs), PROMPTS) == reference()


def test_single_request_matches_batched():
    assert [run(build(), [p])[0] for p in PROMPTS] == reference()


def test_preemption_preserves_output():
    engine = build(block_size=4, num_blocks=24, max_seqs=8, prefix_cache=False)
    got = run(engine, PROMPTS, check_counts=True)
    assert engine.batcher.preemptions > 0
    assert got == reference()


def test_preemption_with_prefix_cache_preserves_output():
    engine = build(block_size=4, num_blocks=24, max_seqs=8, prefix_cache=True)
    got = run(engine, PROMPTS, check_counts=True)
    assert engine.batcher.preemptions > 0
    assert got == reference()


def test_all_blocks_returned_when_idle():
    engine = build(prefix_cache=False)
    run(engine, PROMPTS)
    pool = engine.batcher.pool
    assert pool.num_free == pool.num_blocks
    assert all(r == 0 for r in pool.refs)


def test_prefix_cache_hits_on_repeated_prompt():
    engine = build(block_size=4, prefix_cache=True)
    long = "the same long system prompt that two requests happen to share, word for word"
    run(engine, [long + " one"], max_tokens=4, check_counts=True)
    run(engine, [long + " two"], max_tokens=4, check_counts=True)
    assert engine.batcher.pool.stats()["prefix_hit_rate"] > 0
    assert engine.seqs["req-1"].cached_prefix_tokens >= len(long) - 8


def test_prefix_cache_only_reuses_a_genuinely_matching_prefix():
    engine = build(block_size=4, prefix_cache=True)
    run(engine, ["aaaaaaaaaaaaaaaaaaaaaaaa"], max_tokens=4)
    run(engine, ["bbbbbbbbbbbbbbbbbbbbbbbb"], max_tokens=4)
    assert engine.seqs["req-1"].cached_prefix_tokens == 0


def test_max_tokens_is_respected():
    engine = build()
    rid = engine.add_request("hello there", SamplingParams(max_tokens=7, temperature=0.0, ignore_eos=True))
    while engine.has_work:
        engine.step()
    assert len(engine.seqs[rid].output_token_ids) == 7
    assert engine.seqs[rid].stop_reason == "length"


def test_stop_string_truncates_text():
    engine = build()
    rid = engine.add_request("hello", SamplingParams(max_tokens=40, temperature=0.0, ignore_eos=True))
    while engine.has_work:
        engine.step()
    full = engine.get_text(rid)
    assert len(full) > 3
    stop_at = full[2:4]
    e2 = build()
    rid2 = e2.add_request("hello", SamplingParams(max_tokens=40, temperature=0.0,
                                                  ignore_eos=True, stop=[stop_at]))
    while e2.has_work:
        e2.step()
    assert stop_at not in e2.get_text(rid2)
    assert e2.seqs[rid2].stop_reason == "stop"


def test_abort_frees_the_blocks():
    engine = build()
    rid = engine.add_request("hello there friend", SamplingParams(max_tokens=50, temperature=0.0, ignore_eos=True))
    engine.step()
    engine.step()
    assert engine.abort(rid)
    assert not engine.has_work
    pool = engine.batcher.pool
    assert pool.num_free == pool.num_blocks and pool.audit()


def test_prompt_larger_than_cache_is_rejected_not_hung():
    engine = build(block_size=4, num_blocks=4, max_seqs=2)
    rid = engine.add_request("x" * 400, SamplingParams(max_tokens=5, temperature=0.0, ignore_eos=True))
    outs = []
    for _ in range(50):
        outs += engine.step()
        if not engine.has_work:
            break
    assert not engine.has_work
    assert any(o.request_id == rid and o.finished for o in outs)


def test_seeded_sampling_is_reproducible():
    a, b = build(), build()
    p = SamplingParams(max_tokens=16, temperature=0.9, top_p=0.95, seed=7, ignore_eos=True)
    ra, rb = a.add_request("hello", p), b.add_request("hello", p)
    while a.has_work:
        a.step()
    while b.has_work:
        b.step()
    assert a.seqs[ra].output_token_ids == b.seqs[rb].output_token_ids


def test_sampling_matches_reference_draws():
    """`choose` against the reference's sample() (vllmlite/sampling.py:41-64):
    72 rows whose logits take a few values (ties in most rows), over
    temperature 0/0.7/1/1.3, top_k 0/5/20, top_p 1/0.9/0.5, repetition
    penalty 1/1.3 and the min_tokens EOS mask; three successive draws from
    one seeded generator each, written by the reference
    (tests/golden/make_golden.py)."""
    with open(os.path.join(os.path.dirname(__file__), "golden", "sampling_choices.json")) as f:
        cases = json.load(f)["cases"]
    ties = 0
    for c in cases:
        row = np.array(c["row"], np.float32)
        ties += len(np.unique(row)) < row.size
        p = SamplingParams(temperature=c["temperature"], top_k=c["top_k"], top_p=c["top_p"],
                           repetition_penalty=c["repetition_penalty"],
                           min_tokens=c["min_tokens"], seed=c["seed"])
        g = np.random.default_rng(c["seed"])
        got = [choose(row, p, c["seen"], g, c["num_generated"], c["eos_id"]) for _ in range(3)]
        assert got == c["draws"], c
    assert ties == len(cases)


def test_empty_token_list_rejected():
    with pytest.raises(ValueError):
        build().add_request(params=SamplingParams(), prompt_token_ids=[])


def test_fork_shares_blocks_and_copy_on_write_keeps_streams():
    """fork_request: children share the parent's partial tail block, their
    first write emits CoW pairs (block_manager.py:77-85) and, greedy on the
    same context, they continue exactly as the parent does."""
    engine = build(block_size=4)
    p = SamplingParams(max_tokens=6, temperature=0.0, ignore_eos=True)
    rid = engine.add_request("copy on write please", p)
    engine.step()
    kids = [engine.fork_request(rid, f"kid{i}") for i in range(3)]
    cows = []
    real = engine.runner.execute

    def execute(sched):
        cows.extend(sched.cow)
        return real(sched)

    engine.runner.execute = execute
    while engine.has_work:
        engine.step()
    assert len(cows) == 3 and len({d for _, d in cows}) == 3
    want = engine.seqs[rid].output_token_ids
    assert all(engine.seqs[k].output_token_ids == want for k in kids)
    pool = engine.batcher.pool
    assert pool.num_free == pool.num_blocks and pool.audit()


class _ArgmaxRunner(NumpyRunner):
    """The oracle runner with the argmax entry the HIP runner offers: the same
    rows, reduced by np.argmax; counts the steps that take it."""

    def __init__(self, *a, **kw):
        super().__init__(*a, **kw)
        self.argmax_steps = 0

    def execute_argmax(self, out):
        logits, rows = self.execute(out)
        self.argmax_steps += 1
        return np.argmax(logits, axis=-1).astype(np.int32), rows


def _streams(engine, params_list):
    ids = [engine.add_request(p_, p) for p_, p in params_list]
    while engine.has_work:
        engine.step()
    return [engine.seqs[i].output_token_ids for i in ids]


@pytest.mark.parametrize("spec", [0, 3])
def test_argmax_dispatch_keeps_streams(spec):
    """Greedy steps through execute_argmax give the streams of execute() +
    sampling, with and without draft verification."""
    from vllmlite_amd.speculative import NgramProposer
    rep = PROMPTS + ["abcdefgh abcdefgh abcdefgh abcdefgh abcdefgh"]
    p = SamplingParams(max_tokens=16, temperature=0.0, ignore_eos=True)
    out = []
    for dev in (True, False):
        e = build(runner_factory=_ArgmaxRunner)
        if spec:
            e.spec_k = spec
            e.proposer = NgramProposer(spec)
        e.device_argmax = dev
        out.append(_streams(e, [(x, p) for x in rep]))
        assert (e.runner.argmax_steps > 0) == dev
    assert out[0] == out[1]


def test_argmax_dispatch_falls_back_for_sampled_and_masked_rows():
    """A step holding a sampled, a penalised or an EOS-masked (min_tokens)
    request reads full logits rows; all-greedy steps take the argmax entry."""
    e = build(runner_factory=_ArgmaxRunner)
    assert e.device_argmax
    greedy = SamplingParams(max_tokens=4, temperature=0.0, ignore_eos=True)
    _streams(e, [("hello", greedy)])
    assert e.runner.argmax_steps == e.total_steps
    for p in (SamplingParams(max_tokens=4, temperature=0.8, seed=1),
              SamplingParams(max_tokens=4, temperature=0.0, repetition_penalty=1.3),
              SamplingParams(max_tokens=4, temperature=0.0, min_tokens=8)):
        e = build(runner_factory=_ArgmaxRunner)
        ref = build()
        got = _streams(e, [("hello", greedy), ("the quick brown fox", p)])
        want = _streams(ref, [("hello", greedy), ("the quick brown fox", p)])
        assert got == want
        assert e.runner.argmax_steps == 0

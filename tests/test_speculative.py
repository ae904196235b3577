"""N-gram proposer, greedy verify known answers and speculation invariance
(the reference's tests/test_speculative.py:18-133) on the CPU oracle runner."""

import numpy as np
import pytest

from vllmlite_amd.request import SamplingParams
from vllmlite_amd.speculative import NgramProposer, accept_greedy, verify
from oracle import greedy as oracle_greedy

from helpers import PROMPTS, build, run
from test_engine_invariance import reference

REPETITIVE = [
    "abcdefgh abcdefgh abcdefgh abcdefgh abcdefgh abcdefgh abcdefgh abcdefgh",
    "one two three four one two three four one two three four one two three four",
]


def seq_with(tokens):
    from vllmlite_amd.request import Request
    return Request("t", list(tokens), SamplingParams())


def spec_engine(k, **kw):
    e = build(**kw)
    e.spec_k = k
    e.proposer = NgramProposer(k)
    return e


def test_ngram_finds_the_earlier_continuation():
    assert NgramProposer(k=3, min_n=3, max_n=8).propose(seq_with([1, 2, 3, 9, 8, 7, 1, 2, 3]), 3) == [9, 8, 7]


def test_ngram_returns_nothing_without_a_repeat():
    assert NgramProposer(k=4, min_n=3).propose(seq_with([1, 2, 3, 4, 5, 6, 7, 8]), 4) == []


def test_ngram_prefers_the_longer_match():
    toks = [5, 6, 7, 4, 4, 1, 5, 6, 9, 4, 4, 1, 5, 6]
    assert NgramProposer(k=1, min_n=2, max_n=6).propose(seq_with(toks), 1) == [9]


def _logits_for(picks, vocab=10):
    out = np.full((len(picks), vocab), -5.0, dtype=np.float32)
    for i, t in enumerate(picks):
        out[i, t] = 5.0
    return out


@pytest.mark.parametrize("impl", [verify, oracle_greedy.verify])
def test_verify_known_answers(impl):
    assert impl(_logits_for([3, 4, 5, 6]), [3, 4, 5]) == ([3, 4, 5, 6], 3)
    assert impl(_logits_for([3, 9, 5, 6]), [3, 4, 5]) == ([3, 9], 1)
    assert impl(_logits_for([9, 1, 1]), [3, 4]) == ([9], 0)


def test_verify_ties_go_to_the_lowest_index():
    row = np.zeros((2, 6), np.float32)
    row[:, 2] = row[:, 4] = 1.0
    assert verify(row, [2]) == ([2, 2], 1)
    assert oracle_greedy.verify(row, [2]) == ([2, 2], 1)


def test_accept_greedy_matches_oracle_on_random_rows():
    rng = np.random.default_rng(0)
    for _ in range(200):
        k = int(rng.integers(0, 6))
        logits = rng.standard_normal((k + 1, 7)).astype(np.float32)
        drafts = [int(x) for x in rng.integers(0, 7, size=k)]
        assert accept_greedy(np.argmax(logits, -1), drafts) == oracle_greedy.verify(logits, drafts)


@pytest.mark.parametrize("k", [1, 2, 4, 8])
def test_speculation_does_not_change_the_output(k):
    assert run(spec_engine(k), PROMPTS) == reference()


@pytest.mark.parametrize("k", [2, 4])
def test_speculation_matches_on_repetitive_text(k):
    assert run(spec_engine(k), REPETITIVE, max_tokens=40) == run(build(), REPETITIVE, max_tokens=40)


def test_speculation_cuts_the_number_of_forward_passes():
    plain = build()
    run(plain, REPETITIVE, max_tokens=48)
    fast = spec_engine(6)
    run(fast, REPETITIVE, max_tokens=48)
    assert fast.spec.accepted > 0
    assert fast.total_steps < plain.total_steps


def test_speculation_survives_preemption():
    fast = spec_engine(4, block_size=4, num_blocks=24)
    got = run(fast, PROMPTS, check_counts=True)
    assert fast.batcher.preemptions > 0
    assert got == run(build(block_size=4, num_blocks=24), PROMPTS)


def test_speculation_frees_every_block():
    fast = spec_engine(4)
    run(fast, REPETITIVE, max_tokens=32)
    pool = fast.batcher.pool
    assert pool.num_free == pool.num_blocks and pool.audit()


def test_speculation_respects_max_tokens():
    fast = spec_engine(8)
    rid = fast.add_request(REPETITIVE[0], SamplingParams(max_tokens=5, temperature=0.0, ignore_eos=True))
    while fast.has_work:
        fast.step()
    assert len(fast.seqs[rid].output_token_ids) == 5


def test_stats_report_acceptance():
    fast = spec_engine(4)
    run(fast, REPETITIVE, max_tokens=32)
    s = fast.stats()
    assert 0.0 < s["spec_acceptance_rate"] <= 1.0
    assert s["spec_tokens_per_step"] > 1.0

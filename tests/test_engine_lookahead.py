"""Lookahead stepping (the engine launches step n + 1 before it has step n's
tokens) reproduces synchronous stepping: the reference's streams, step counts
and prefix-cache behaviour, on the CPU with the oracle runner.

`_LaunchingRunner` gives the oracle runner the launch / collect interface of
HipRunner and resolves a placeholder token id t < 0 to row -t - 1 of the
previous launch's argmax, as vl_resolve_tokens does on the device."""

import json
import os

import numpy as np
import pytest

from oracle.runner import NumpyRunner
from vllmlite_amd.engine import LLMEngine
from vllmlite_amd.request import SamplingParams
from vllmlite_amd.workload import mixed_lengths, shared_prefix_config

from helpers import PROMPTS, cfg0_config, run, small_cfg

GOLD = os.path.join(os.path.dirname(__file__), "golden")


class _LaunchingRunner(NumpyRunner):
    def __init__(self, *a, **kw):
        super().__init__(*a, **kw)
        self.prev = np.zeros(0, np.int32)
        self.launches = 0
        self.placeholders = 0

    def execute_argmax(self, out):
        return self.collect(self.launch_argmax(out))

    def launch_argmax(self, out):
        for item in out.scheduled:
            ids = item.seq.ids
            for pos in range(item.start_pos, item.start_pos + item.num_tokens):
                if ids[pos] < 0:
                    self.placeholders += 1
                    ids[pos] = int(self.prev[-ids[pos] - 1])
        logits, rows = self.execute(out)
        self.prev = np.argmax(logits, axis=-1).astype(np.int32)
        self.launches += 1
        return rows, self.prev.copy()

    def collect(self, handle):
        rows, ids = handle
        return ids, rows


def _drive(cfg, reqs, lookahead):
    eng = LLMEngine(cfg, runner=_LaunchingRunner(cfg.model, cfg.cache), lookahead=lookahead)
    for rid, ids, p in reqs:
        eng.add_request(params=p, request_id=rid, prompt_token_ids=ids)
    outs = []
    while eng.has_work:
        outs += eng.step()
    return eng, outs


def _load(name):
    with open(os.path.join(GOLD, name)) as f:
        return json.load(f)


def test_lookahead_mix_matches_reference_streams_and_steps():
    g = _load("cfg0_streams.json")
    eng, outs = _drive(cfg0_config(False), mixed_lengths(0, 48, 0), True)
    assert eng.runner.placeholders > 1000  # the pipeline was in use
    assert eng.total_steps == g["steps"] == 260
    for rid in g["streams"]:
        assert eng.seqs[rid].output_token_ids == g["streams"][rid], rid
    # every emitted token was reported once, in order, with the final output
    per = {}
    for o in outs:
        per.setdefault(o.request_id, []).extend(o.new_token_ids)
    assert per == g["streams"]
    assert all(o.finish_reason == "length" for o in outs if o.finished)


def test_lookahead_with_prefix_cache_matches_reference():
    """Blocks are published from committed tokens only: placeholders are
    replaced before the next step's commit, so prefix hits, the 280 steps and
    the streams are the reference's."""
    g = _load("shared_prefix_streams.json")["plain"]
    eng, _ = _drive(shared_prefix_config(True), mixed_lengths(0, 48, 256), True)
    assert eng.total_steps == g["steps"] == 280
    assert eng.stats()["prefix_hit_rate"] == 1.0
    for rid in g["streams"]:
        assert eng.seqs[rid].output_token_ids == g["streams"][rid], rid
    assert eng.batcher.pool.audit()


def test_lookahead_under_preemption_and_small_blocks():
    """A squeezed cache (block 4, 24 blocks) preempts requests whose last token
    is still a placeholder; their recompute takes it from the device."""
    p = SamplingParams(max_tokens=20, temperature=0.0, ignore_eos=True)
    want = _load("small_streams.json")["streams"]
    for prefix in (False, True):
        cfg = small_cfg(block_size=4, num_blocks=24, max_seqs=8, prefix_cache=prefix)
        eng = LLMEngine(cfg, runner=_LaunchingRunner(cfg.model, cfg.cache))
        ids = [eng.add_request(x, p) for x in PROMPTS]
        while eng.has_work:
            eng.step()
            assert eng.batcher.pool.audit()
        assert eng.batcher.preemptions > 0
        assert [eng.seqs[i].output_token_ids for i in ids] == want


@pytest.mark.parametrize("params,looked_ahead", [
    (SamplingParams(max_tokens=8, temperature=0.0), False),   # an EOS may stop it
    (SamplingParams(max_tokens=8, temperature=0.0, ignore_eos=True, stop=["zz"]), False),
    # EOS masked for the first 4 tokens: those steps are synchronous, the rest not
    (SamplingParams(max_tokens=8, temperature=0.0, ignore_eos=True, min_tokens=4), True),
    (SamplingParams(max_tokens=8, temperature=0.7, seed=3, ignore_eos=True), False),
])
def test_value_dependent_steps_run_synchronously(params, looked_ahead):
    """Steps whose outcome can depend on the chosen tokens are not looked
    ahead; every stream equals the synchronous engine's."""
    streams = []
    for lookahead in (True, False):
        cfg = small_cfg()
        eng = LLMEngine(cfg, runner=_LaunchingRunner(cfg.model, cfg.cache), lookahead=lookahead)
        ids = [eng.add_request(x, params) for x in PROMPTS]
        while eng.has_work:
            eng.step()
        streams.append([eng.seqs[i].output_token_ids for i in ids])
        if lookahead:
            assert (eng.runner.placeholders > 0) == looked_ahead
    assert streams[0] == streams[1]


def test_lookahead_off_is_synchronous():
    cfg = small_cfg()
    eng = LLMEngine(cfg, runner=_LaunchingRunner(cfg.model, cfg.cache), lookahead=False)
    assert run(eng, PROMPTS) == _load("small_streams.json")["streams"]
    assert eng.runner.placeholders == 0


def test_fork_refuses_while_a_step_is_in_flight():
    cfg = small_cfg()
    eng = LLMEngine(cfg, runner=_LaunchingRunner(cfg.model, cfg.cache))
    rid = eng.add_request("copy on write please",
                          SamplingParams(max_tokens=6, temperature=0.0, ignore_eos=True))
    eng.step()
    with pytest.raises(RuntimeError):
        eng.fork_request(rid, "kid")


def _reports(outs):
    """Per request: every token reported, and each finished report's
    (reason, token_ids)."""
    toks, fins = {}, {}
    for o in outs:
        assert all(t >= 0 for t in o.token_ids), o  # no placeholder leaks out
        toks.setdefault(o.request_id, []).extend(o.new_token_ids)
        if o.finished:
            fins.setdefault(o.request_id, []).append((o.finish_reason, list(o.token_ids)))
    return toks, fins


def _drive_with_abort(lookahead, victim_params, abort_after, check):
    """Request a (greedy, ignore_eos) runs; request b joins after two steps;
    b is aborted after `abort_after` more calls; both engines see the same
    sequence of calls."""
    cfg = small_cfg()
    eng = LLMEngine(cfg, runner=_LaunchingRunner(cfg.model, cfg.cache), lookahead=lookahead)
    greedy = SamplingParams(max_tokens=12, temperature=0.0, ignore_eos=True)
    outs = []
    eng.add_request(PROMPTS[0], greedy, request_id="a")
    outs += eng.step()
    outs += eng.step()
    eng.add_request(PROMPTS[1], victim_params, request_id="b")
    for _ in range(abort_after):
        outs += eng.step()
    if lookahead:
        check(eng)
    assert eng.abort("b")
    while eng.has_work:
        outs += eng.step()
        assert eng.batcher.pool.audit()
    return eng, outs


def test_abort_of_a_request_held_for_a_synchronous_step():
    """A sampled request joins while a greedy step is in flight: the next batch
    is held for a synchronous step; aborting the sampled request before that
    step drops it from the held batch (its blocks are already free)."""
    sampled = SamplingParams(max_tokens=12, temperature=0.7, seed=5, ignore_eos=True)
    runs = [_drive_with_abort(la, sampled, 1, lambda e: e._next is not None and any(
        i.seq.request_id == "b" for i in e._next.scheduled)) for la in (True, False)]
    (eng, outs), (ref, ref_outs) = runs
    assert eng.seqs["a"].output_token_ids == ref.seqs["a"].output_token_ids
    toks, fins = _reports(outs)
    rfins = _reports(ref_outs)[1]
    assert fins["a"] == rfins["a"]
    assert toks["a"] == eng.seqs["a"].output_token_ids
    # b never ran under lookahead (its first step was the held one); the
    # synchronous engine had run its prefill by the same call
    assert fins["b"] == [("abort", [])] and rfins["b"][0][0] == "abort"


@pytest.mark.parametrize("abort_after", [1, 2, 3])
def test_abort_while_its_step_is_in_flight(abort_after):
    """Aborting a greedy request whose step is on the device: its in-flight
    token is reported (as synchronous stepping reported it before the abort),
    then one finished report with the real ids and reason "abort"."""
    greedy = SamplingParams(max_tokens=12, temperature=0.0, ignore_eos=True)
    eng, outs = _drive_with_abort(True, greedy, abort_after, lambda e: e._inflight is not None)
    ref, ref_outs = _drive_with_abort(False, greedy, abort_after, lambda e: None)
    toks, fins = _reports(outs)
    rtoks, rfins = _reports(ref_outs)
    assert len(fins["b"]) == 1 and fins["b"][0][0] == "abort"
    assert fins["b"][0][1] == eng.seqs["b"].output_token_ids == toks["b"]
    assert eng.seqs["a"].output_token_ids == ref.seqs["a"].output_token_ids == toks["a"]
    assert fins["a"] == rfins["a"]
    # the looked-ahead engine has one more step of b on the device when the
    # abort lands; what it reports of b is a prefix of b's greedy stream
    assert rtoks["b"] == toks["b"][:len(rtoks["b"])]


def test_cache_full_retirement_under_lookahead():
    """A request that outgrows a 4-block cache is retired "cache_full" by the
    schedule that follows its in-flight step: one finished report, after the
    in-flight token, with real ids, as synchronous stepping gives."""
    got = []
    for lookahead in (True, False):
        cfg = small_cfg(block_size=4, num_blocks=4)
        eng = LLMEngine(cfg, runner=_LaunchingRunner(cfg.model, cfg.cache), lookahead=lookahead)
        eng.add_request(params=SamplingParams(max_tokens=64, temperature=0.0, ignore_eos=True),
                        request_id="r", prompt_token_ids=[1, 72, 101, 108, 108])
        outs = []
        while eng.has_work:
            outs += eng.step()
        if lookahead:
            assert eng.runner.placeholders > 0
        got.append(_reports(outs))
    assert got[0] == got[1]
    fins = got[0][1]["r"]
    assert len(fins) == 1 and fins[0][0] == "cache_full"

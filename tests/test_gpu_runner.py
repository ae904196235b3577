"""HipRunner behind the unchanged engine: greedy streams equal the reference's
and are invariant to paging, chunking, batching, prefix caching, preemption
and speculation (the reference's tests/test_engine.py:57-204 and
tests/test_speculative.py:63-101), with the expected streams taken from the
reference itself (tests/golden/*.json).

Bar: identical greedy token streams, except at an argmax near-tie. A
divergence is accepted only where the reference's own top-1/top-2 logit margin
at that token is below NEAR_TIE (fp32 reductions in a different order move
logits by ~1e-6 relative); every other difference fails.
"""

import json
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from vllmlite_amd.engine import LLMEngine  # noqa: E402
from vllmlite_amd.speculative import NgramProposer  # noqa: E402
from vllmlite_amd.workload import mixed_lengths  # noqa: E402

from helpers import PROMPTS, cfg0_config, run, small_cfg  # noqa: E402

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")
NEAR_TIE = 1e-4


def _gold(name):
    with open(os.path.join(GOLD, name)) as f:
        return json.load(f)


def hip_engine(use_graphs=True, **kw):
    from vllmlite_amd.hip_runner import HipRunner
    cfg = small_cfg(**kw)
    return LLMEngine(cfg, runner=HipRunner(cfg.model, cfg.cache, use_graphs=use_graphs))


def small_reference():
    g = _gold("small_streams.json")
    assert g["prompts"] == PROMPTS
    return g["streams"]


@pytest.mark.parametrize("layout", ["token", "head"])
def test_cfg0_mix_matches_reference_streams(layout):
    """The 48-request ragged mix end to end: 260 steps, 3179 tokens, the
    reference's greedy streams token for token (near-ties excepted), with
    the cache token-major (the reference's layout) or head-major."""
    from vllmlite_amd.hip_runner import HipRunner
    g = _gold("cfg0_streams.json")
    cfg = cfg0_config(False)
    cfg.cache.kv_layout = layout
    eng = LLMEngine(cfg, runner=HipRunner(cfg.model, cfg.cache))
    reqs = mixed_lengths(0, 48, 0)
    for rid, ids, p in reqs:
        eng.add_request(params=p, request_id=rid, prompt_token_ids=ids)
    while eng.has_work:
        eng.step()
    diverged = []
    for rid, _, _ in reqs:
        got, want = eng.seqs[rid].output_token_ids, g["streams"][rid]
        assert len(got) == len(want), rid
        for j, (a, b) in enumerate(zip(got, want)):
            if a != b:
                diverged.append((rid, j, g["margins"][rid][j]))
                break
    for rid, j, margin in diverged:
        assert margin < NEAR_TIE, f"{rid} diverges at token {j} with reference margin {margin}"
    assert eng.total_steps == g["steps"] == 260
    print("diverged at near-ties:", diverged)


def test_default_engine_matches_reference_streams():
    assert run(hip_engine(), PROMPTS, check_counts=True) == small_reference()


def test_graph_replay_equals_eager_logits():
    """Every step's logits from HIP-graph replay are bitwise those of eager runs."""
    a, b = hip_engine(use_graphs=True), hip_engine(use_graphs=False)
    seen = []
    for eng in (a, b):
        logs = []
        real = eng.runner.execute

        def execute(sched, real=real, logs=logs):
            lg, rows = real(sched)
            logs.append(lg.copy())
            return lg, rows

        eng.runner.execute = execute
        eng.device_argmax = False  # every step through execute()
        run(eng, PROMPTS)
        seen.append(logs)
    assert len(seen[0]) == len(seen[1])
    for x, y in zip(*seen):
        assert np.array_equal(x, y)


@pytest.mark.parametrize("block_size", [1, 4, 16, 64])
def test_block_size_does_not_change_output(block_size):
    assert run(hip_engine(block_size=block_size), PROMPTS) == small_reference()


def test_prefix_caching_does_not_change_output():
    assert run(hip_engine(prefix_cache=True), PROMPTS, check_counts=True) == small_reference()


@pytest.mark.parametrize("max_batched", [8, 33, 64, 4096])
def test_chunked_prefill_does_not_change_output(max_batched):
    assert run(hip_engine(max_batched=max_batched), PROMPTS) == small_reference()


def test_no_chunked_prefill_matches():
    assert run(hip_engine(chunked=False, max_batched=4096), PROMPTS) == small_reference()


@pytest.mark.parametrize("max_seqs", [1, 2, 3, 8])
def test_batch_composition_does_not_change_output(max_seqs):
    assert run(hip_engine(max_seqs=max_seqs), PROMPTS) == small_reference()


def test_single_request_matches_batched():
    from vllmlite_amd.hip_runner import HipRunner
    cfg = small_cfg()
    runner = HipRunner(cfg.model, cfg.cache)  # one runner (and its graphs) for every engine
    solo = [run(LLMEngine(cfg, runner=runner), [p])[0] for p in PROMPTS]
    assert solo == small_reference()


@pytest.mark.parametrize("prefix_cache", [False, True])
def test_preemption_preserves_output(prefix_cache):
    engine = hip_engine(block_size=4, num_blocks=24, max_seqs=8, prefix_cache=prefix_cache)
    got = run(engine, PROMPTS, check_counts=True)
    assert engine.batcher.preemptions > 0
    assert got == small_reference()


@pytest.mark.parametrize("k", [1, 2, 4, 8])
def test_speculation_does_not_change_the_output(k):
    e = hip_engine()
    e.spec_k = k
    e.proposer = NgramProposer(k)
    assert run(e, PROMPTS) == small_reference()


@pytest.mark.parametrize("k", [1, 4])
def test_speculation_matches_plain_greedy(k):
    e = hip_engine()
    e.spec_k = k
    e.proposer = NgramProposer(k)
    rep = ["abcdefgh abcdefgh abcdefgh abcdefgh abcdefgh abcdefgh abcdefgh abcdefgh"]
    plain = run(hip_engine(), rep, max_tokens=40)
    assert run(e, rep, max_tokens=40) == plain
    assert e.spec.accepted > 0


@pytest.mark.parametrize("k", [0, 4])
def test_device_argmax_matches_host_argmax(k):
    """Greedy steps through execute_argmax / launch_argmax (argmax on the
    device, R int32 values to the host) give the streams of execute() +
    np.argmax, with and without draft verification; the device path is the
    one taken."""
    rep = PROMPTS + ["abcdefgh abcdefgh abcdefgh abcdefgh abcdefgh abcdefgh"]
    streams, calls = [], []
    for dev in (True, False):
        e = hip_engine()
        if k:
            e.spec_k = k
            e.proposer = NgramProposer(k)
        e.device_argmax = dev
        n = [0]
        for name in ("execute_argmax", "launch_argmax"):
            real = getattr(e.runner, name)

            def counted(sched, real=real, n=n):
                n[0] += 1
                return real(sched)

            setattr(e.runner, name, counted)
        streams.append(run(e, rep, max_tokens=24))
        calls.append(n[0])
    assert streams[0] == streams[1]
    assert calls[0] > 0 and calls[1] == 0


def test_device_argmax_ids_equal_numpy_argmax():
    """execute_argmax returns np.argmax of execute()'s rows for the same step
    (the forward is deterministic: graph replay is bitwise eager)."""
    e = hip_engine()
    e.lookahead = False  # every greedy step through execute_argmax
    got = []
    real_x, real_a = e.runner.execute, e.runner.execute_argmax

    def execute_argmax(sched):
        ids, rows = real_a(sched)
        lg, rows2 = real_x(sched)
        assert rows == rows2
        got.append((ids, np.argmax(lg, axis=-1).astype(np.int32)))
        return ids, rows

    e.runner.execute_argmax = execute_argmax
    run(e, PROMPTS, max_tokens=8)
    assert got
    for ids, want in got:
        assert np.array_equal(ids, want)


@pytest.mark.parametrize("layout", ["token", "head"])
def test_copy_on_write_fork_matches_oracle_runner(layout):
    """A forked parent with a partial tail block: the children's first decode
    step writes into the shared block, so the block manager emits CoW pairs;
    the HipRunner's streams (either cache layout) must match the NumPy oracle
    runner's."""
    from oracle.runner import NumpyRunner
    from vllmlite_amd.hip_runner import HipRunner
    from vllmlite_amd.request import SamplingParams

    cfg = small_cfg(block_size=4)
    cfg.cache.kv_layout = layout
    outs = []
    for factory in (NumpyRunner, HipRunner):
        eng = LLMEngine(cfg, runner=factory(cfg.model, cfg.cache), lookahead=False)
        p = SamplingParams(max_tokens=6, temperature=0.0, ignore_eos=True)
        rid = eng.add_request("copy on write please", p)
        eng.step()  # prefill: 20 tokens -> a partial 6th block
        kids = [eng.fork_request(rid, f"kid{i}") for i in range(3)]
        cows = []
        real = eng.runner.execute

        def execute(sched, real=real, cows=cows):
            cows.extend(sched.cow)
            return real(sched)

        eng.runner.execute = execute
        eng.device_argmax = False  # every step through execute()
        while eng.has_work:
            eng.step()
        assert cows, "no copy-on-write pair was scheduled"
        outs.append([eng.seqs[r].output_token_ids for r in [rid] + kids])
    assert outs[0] == outs[1]


def _cfg3_engine(fork_counts=None):
    from vllmlite_amd.hip_runner import HipRunner
    from vllmlite_amd.workload import shared_prefix_config
    cfg = shared_prefix_config(True)
    eng = LLMEngine(cfg, runner=HipRunner(cfg.model, cfg.cache))
    if fork_counts is not None:
        for name in ("execute", "execute_argmax"):
            real = getattr(eng.runner, name)

            def counting(out, real=real):
                fork_counts.extend(out.cow)
                return real(out)

            setattr(eng.runner, name, counting)
    return eng


def test_shared_prefix_mix_matches_reference_streams():
    """48 requests behind a 256-token system prompt with the prefix cache on
    (prefill skips the cached blocks): the reference's 280 steps and streams."""
    g = _gold("shared_prefix_streams.json")
    eng = _cfg3_engine()
    reqs = mixed_lengths(0, 48, 256)
    for rid, ids, p in reqs:
        eng.add_request(params=p, request_id=rid, prompt_token_ids=ids)
    while eng.has_work:
        eng.step()
    assert eng.total_steps == g["plain"]["steps"] == 280
    same = sum(eng.seqs[rid].output_token_ids == g["plain"]["streams"][rid] for rid, _, _ in reqs)
    assert same == 48


def test_forked_shared_prefix_copy_on_write_matches_reference():
    """The same mix with every request forked after its first token: 44
    copy-on-write pairs (one per partial shared tail, 4 prompts end on a block
    boundary) run through vl_copy_blocks, and every parent's and child's
    stream, the step count and the pair count equal the reference's."""
    from vllmlite_amd.workload import drive_forked
    g = _gold("shared_prefix_streams.json")["forked"]
    pairs = []
    eng = _cfg3_engine(pairs)
    forked, partial = drive_forked(eng, mixed_lengths(0, 48, 256))
    assert partial == g["partial_tails"] and len(pairs) == g["cow_pairs"] == 44
    assert eng.total_steps == g["steps"]
    got = {rid: s.output_token_ids for rid, s in eng.seqs.items()}
    assert sorted(got) == sorted(g["streams"])
    bad = [rid for rid in got if got[rid] != g["streams"][rid]]
    assert not bad, f"streams differ: {bad[:5]}"


def _logit_trace(runner_factory, cfg, prompts, max_tokens):
    """Logits of every step (through execute()) of a greedy run."""
    eng = LLMEngine(cfg, runner=runner_factory(cfg.model, cfg.cache))
    eng.device_argmax = False
    logs = []
    real = eng.runner.execute

    def execute(sched, real=real):
        lg, rows = real(sched)
        logs.append((lg.copy(), all(i.num_tokens == 1 for i in sched.scheduled)))
        return lg, rows

    eng.runner.execute = execute
    run(eng, prompts, max_tokens=max_tokens)
    return logs


@pytest.mark.parametrize("layers,d_model", [(2, 64), (6, 384)])
def test_every_step_logits_match_oracle_runner(layers, d_model):
    """Every step's logits, prefill steps (GEMM path) and single-token decode
    steps (fused projection kernels) alike, against the NumPy oracle runner's
    (vllmlite/model.py:80-120): within 2e-4 of each row's largest logit (fp32
    sums in a different order)."""
    from oracle.runner import NumpyRunner
    from vllmlite_amd.hip_runner import HipRunner
    cfg = small_cfg(layers=layers, d_model=d_model)
    if d_model == 384:  # the TinyLlama mix's shape
        cfg.model.n_heads, cfg.model.n_kv_heads, cfg.model.d_ff = 8, 4, 1024
    got = _logit_trace(HipRunner, cfg, PROMPTS, 12)
    want = _logit_trace(NumpyRunner, cfg, PROMPTS, 12)
    assert len(got) == len(want) and sum(dec for _, dec in got) >= 10
    for (g, dec), (w, _) in zip(got, want):
        scale = np.abs(w).max(axis=-1, keepdims=True)
        assert np.all(np.abs(g - w) <= 2e-4 * scale), f"decode step {dec}"


@pytest.mark.parametrize("layers,d_model", [(2, 64), (6, 384)])
def test_head_major_cache_gives_the_same_logits(layers, d_model):
    """cache kv_layout "head" ([blocks, Hkv, block_size, D] per layer): every
    step's logits, prefill and decode, equal those with the token-major cache
    bit for bit (the kernels read the same values in the same order; only the
    addresses differ)."""
    from vllmlite_amd.hip_runner import HipRunner
    traces = []
    for layout in ("token", "head"):
        cfg = small_cfg(layers=layers, d_model=d_model)
        if d_model == 384:
            cfg.model.n_heads, cfg.model.n_kv_heads, cfg.model.d_ff = 8, 4, 1024
        cfg.cache.kv_layout = layout
        traces.append(_logit_trace(HipRunner, cfg, PROMPTS, 12))
    assert len(traces[0]) == len(traces[1]) and sum(dec for _, dec in traces[0]) >= 10
    for (a, _), (b, _) in zip(*traces):
        assert np.array_equal(a, b)


def test_runner_reads_weights_from_npz(tmp_path):
    """HipRunner with model.weights_path (vllmlite/runner.py:41-44,
    model.py:60-71) computes with the file's weights: every step's logits
    equal those of a HipRunner handed the same weights directly, bit for bit,
    and the oracle runner's with them within 2e-4 of each row's largest."""
    import dataclasses
    from oracle.runner import NumpyRunner
    from vllmlite_amd.hip_runner import HipRunner
    from vllmlite_amd.model import init_weights
    cfg = small_cfg()
    other = init_weights(dataclasses.replace(cfg.model, seed=7))
    path = tmp_path / "w.npz"
    np.savez(path, **other)
    cfg_file = small_cfg()
    cfg_file.model = dataclasses.replace(cfg_file.model, weights_path=str(path))
    got = _logit_trace(HipRunner, cfg_file, PROMPTS[:2], 6)
    direct = _logit_trace(lambda m, c: HipRunner(m, c, weights=other), cfg, PROMPTS[:2], 6)
    want = _logit_trace(lambda m, c: NumpyRunner(m, c, weights=other), cfg, PROMPTS[:2], 6)
    seeded = _logit_trace(HipRunner, cfg, PROMPTS[:2], 6)
    assert len(got) == len(direct) == len(want)
    assert not np.array_equal(got[0][0], seeded[0][0])  # the file, not the seed
    for (g, _), (d, _), (w, _) in zip(got, direct, want):
        assert np.array_equal(g, d)
        assert np.all(np.abs(g - w) <= 2e-4 * np.abs(w).max(axis=-1, keepdims=True))


@pytest.mark.parametrize("layers,d_model", [(2, 64), (6, 384)])
def test_bf16_kv_cache_logits_match_oracle_runner(layers, d_model):
    """cache kv_dtype "bfloat16": every step's logits against the oracle
    runner whose cache rounds K/V to bf16 the same way, within 1e-3 of each
    row's largest logit. The fp32 bar (2e-4) does not carry over: K/V
    computed with sums in another order can land one bf16 step (2^-8
    relative) apart when they straddle a rounding midpoint; measured worst
    3.6e-4 on the 6-layer shape, 4e-6 on the 2-layer one."""
    from oracle.runner import NumpyRunner
    from vllmlite_amd.hip_runner import HipRunner
    cfg = small_cfg(layers=layers, d_model=d_model)
    cfg.cache.kv_dtype = "bfloat16"
    if d_model == 384:
        cfg.model.n_heads, cfg.model.n_kv_heads, cfg.model.d_ff = 8, 4, 1024
    got = _logit_trace(HipRunner, cfg, PROMPTS, 12)
    want = _logit_trace(NumpyRunner, cfg, PROMPTS, 12)
    assert len(got) == len(want) and sum(dec for _, dec in got) >= 10
    worst = [float((np.abs(g - w) / np.abs(w).max(axis=-1, keepdims=True)).max())
             for (g, _), (w, _) in zip(got, want)]
    print("worst logit error per step (fraction of the row's largest):",
          [f"{x:.1e}" for x in worst])
    for (g, dec), (w, _) in zip(got, want):
        scale = np.abs(w).max(axis=-1, keepdims=True)
        assert np.all(np.abs(g - w) <= 1e-3 * scale), f"decode step {dec}"


def _narrow_cache_streams(kv_dtype):
    """The 48-request mix with a narrow K/V cache through HipRunner and through
    the oracle runner with the same cache: both runs' streams, and for the
    oracle's, the top-1 minus top-2 logit margin of every emitted token as a
    fraction of its row's largest |logit|."""
    from oracle.runner import NumpyRunner
    from vllmlite_amd.hip_runner import HipRunner
    reqs = mixed_lengths(0, 48, 0)
    streams, margins = {}, {rid: [] for rid, _, _ in reqs}
    for name, factory in (("hip", HipRunner), ("oracle", NumpyRunner)):
        cfg = cfg0_config(False)
        cfg.cache.kv_dtype = kv_dtype
        eng = LLMEngine(cfg, runner=factory(cfg.model, cfg.cache))
        if name == "oracle":
            real = eng.runner.execute
            seen = {}

            def execute(sched, real=real, seen=seen):
                lg, rows = real(sched)
                seen["step"] = (sched, lg, rows)
                return lg, rows

            eng.runner.execute = execute
        for rid, ids, p in reqs:
            eng.add_request(params=p, request_id=rid, prompt_token_ids=ids)
        while eng.has_work:
            before = {rid: len(s.output_token_ids) for rid, s in eng.seqs.items()}
            eng.step()
            if name == "oracle" and "step" in seen:
                sched, lg, rows = seen.pop("step")
                for i, item in enumerate(sched.scheduled):
                    rid = item.seq.request_id
                    if len(eng.seqs[rid].output_token_ids) > before[rid]:
                        row0, c = rows[i]
                        r = lg[row0 + c - 1].astype(np.float64)
                        top = np.sort(r)
                        margins[rid].append((top[-1] - top[-2]) / np.abs(r).max())
        streams[name] = {rid: eng.seqs[rid].output_token_ids for rid, _, _ in reqs}
    return reqs, streams, margins


def _check_divergences(reqs, streams, margins, bound, what):
    """Every stream equals the oracle runner's, except where the oracle's own
    margin at the first differing token is below `bound` (a near-tie that
    logits within the cache's bar can reorder). Returns the divergences."""
    ref = _gold("cfg0_streams.json")["streams"]
    parted = []
    for rid, _, _ in reqs:
        got, want = streams["hip"][rid], streams["oracle"][rid]
        assert len(got) == len(want), rid
        j = next((k for k, (a, b) in enumerate(zip(got, want)) if a != b), None)
        if j is not None:
            parted.append((rid, j, margins[rid][j]))
    as_ref = sum(streams["hip"][r] == ref[r] for r, _, _ in reqs)
    print(f"{what} K/V cache: {len(reqs) - len(parted)}/48 streams equal to the oracle runner's "
          f"with the same cache, {as_ref}/48 to the fp32 reference's; divergences "
          f"(request, token, oracle margin / row max): {parted}")
    for rid, j, m in parted:
        assert m < bound, f"{rid} parts at token {j} where the oracle's margin is {m:.2e}"
    return parted


def test_bf16_kv_cache_mix_streams():
    """The 48-request mix with a bf16 K/V cache: every stream equals the
    oracle runner's with the same bf16 cache, except at a near-tie: a stream
    may part only at a token whose top-1 / top-2 margin in the oracle's
    logits is below 2e-3 of the row's largest |logit| (twice the per-logit
    bar of the bf16 cache, test_bf16_kv_cache_logits_match_oracle_runner).
    How many stay identical to the fp32 reference's streams is printed."""
    _check_divergences(*_narrow_cache_streams("bfloat16"), 2e-3, "bf16")


@pytest.mark.parametrize("layers,d_model", [(2, 64), (6, 384)])
def test_fp8_kv_cache_logits_match_oracle_runner(layers, d_model):
    """cache kv_dtype "float8_e4m3": every step's logits against the oracle
    runner whose cache rounds K/V to FP8 E4M3 the same way, within 1e-3 of
    each row's largest logit, the bf16 cache's bar. A K/V value computed with
    sums in another order can land one FP8 step (2^-3 relative) apart when it
    straddles a rounding midpoint; measured worst 9.9e-5 on the 6-layer
    shape, 3.8e-5 on the 2-layer one."""
    from oracle.runner import NumpyRunner
    from vllmlite_amd.hip_runner import HipRunner
    cfg = small_cfg(layers=layers, d_model=d_model)
    cfg.cache.kv_dtype = "float8_e4m3"
    if d_model == 384:
        cfg.model.n_heads, cfg.model.n_kv_heads, cfg.model.d_ff = 8, 4, 1024
    got = _logit_trace(HipRunner, cfg, PROMPTS, 12)
    want = _logit_trace(NumpyRunner, cfg, PROMPTS, 12)
    assert len(got) == len(want) and sum(dec for _, dec in got) >= 10
    worst = [float((np.abs(g - w) / np.abs(w).max(axis=-1, keepdims=True)).max())
             for (g, _), (w, _) in zip(got, want)]
    print("worst logit error per step (fraction of the row's largest):",
          [f"{x:.1e}" for x in worst])
    assert max(worst) <= 1e-3


def test_fp8_kv_cache_mix_streams():
    """The 48-request mix with an FP8 E4M3 K/V cache: every stream equals the
    oracle runner's with the same FP8 cache, except at a near-tie (the
    oracle's top-1 / top-2 margin below 2e-3 of the row's largest |logit|,
    twice the FP8 cache's per-logit bar). FP8 keeps 3 mantissa bits, so a
    last-bit fp32 difference between two summation orders of a projection
    (the oracle's BLAS and the MFMA kernels) now and then lands a cache
    element on the other side of a rounding boundary, a whole FP8 step, and
    can move a later near-tie. How many stay identical to the fp32 reference
    streams is printed (FP8 keys and values move the logits far more than
    bf16 ones)."""
    _check_divergences(*_narrow_cache_streams("float8_e4m3"), 2e-3, "FP8")


def test_lookahead_across_buffer_growth():
    from vllmlite_amd.request import SamplingParams
    """A launched step whose ids are still on their way to the host while the
    next step grows the runner's buffers (a 2-sequence engine admitting a long
    prompt after short ones): every stream equals the synchronous engine's."""
    p = SamplingParams(max_tokens=12, temperature=0.0, ignore_eos=True)
    prompts = ["hi", "yo", "x" * 150, "a somewhat longer prompt " * 4]
    got = []
    for lookahead in (True, False):
        from vllmlite_amd.hip_runner import HipRunner
        cfg = small_cfg(max_seqs=2)
        eng = LLMEngine(cfg, runner=HipRunner(cfg.model, cfg.cache), lookahead=lookahead)
        ids = [eng.add_request(x, p) for x in prompts]
        while eng.has_work:
            eng.step()
        got.append([eng.seqs[i].output_token_ids for i in ids])
    assert got[0] == got[1]


def test_steps_from_rotating_worker_threads():
    """The reference's async engine calls engine.step through
    run_in_executor (vllmlite/async_engine.py:38-53), so each step may run on
    another thread. Three single-thread executors take the steps of the
    48-request mix in turn: with the lookahead, a step launched on one thread
    is collected on the next. First with a fresh runner (its graphs captured
    on worker threads), then again with the same runner from other workers
    (graphs captured on one thread, replayed on others). Streams equal the
    reference's both times."""
    from concurrent.futures import ThreadPoolExecutor

    from vllmlite_amd.hip_runner import HipRunner
    g = _gold("cfg0_streams.json")
    cfg = cfg0_config(False)
    runner = HipRunner(cfg.model, cfg.cache)
    for rotation in range(2):
        pools = [ThreadPoolExecutor(max_workers=1) for _ in range(3)]
        try:
            threads = set()
            eng = LLMEngine(cfg, runner=runner)
            for rid, ids, p in mixed_lengths(0, 48, 0):
                eng.add_request(params=p, request_id=rid, prompt_token_ids=ids)
            k = 0

            def step():
                import threading
                threads.add(threading.get_ident())
                return eng.step()

            while eng.has_work:
                pools[(k + rotation) % 3].submit(step).result()
                k += 1
            assert len(threads) == 3 and eng.total_steps == g["steps"]
            for rid, want in g["streams"].items():
                assert eng.seqs[rid].output_token_ids == want, (rotation, rid)
        finally:
            for p in pools:
                p.shutdown()

#!/usr/bin/env python3
"""Benchmark of the ragged paged-attention step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-e2e]
                    [--legs decode,mixed,verify,cow,e2e] [--profile-mode LEG]
                    [--copy-only]

The headline (`value`) is the 256-sequence ragged decode batch: 256 sequences
of one query token, context lognormal (median 1024, sigma 0.6) clipped to
64..8192, 32 query heads over 8 KV heads, head_dim 128, bf16 Q/K/V ~N(0,1),
block size 16, block tables drawn as consecutive slices of a seeded
permutation of a 2^17-block pool (8.6 GB of K/V; every slot a sequence does
not own is NaN). A step is one paged-attention run over that batch with the
inputs resident in HBM; the work plan is built once outside the timed region,
as the runner does once per step for all of a model's layers.

One JSON line:
  value         algorithmic HBM bytes per step / step time (GB/s); the step time
                is the host clock over `steps` launches issued back to back,
                between two stream synchronisations
  roofline      the decode launch's average duration from HIP events on the
                stream it is launched on; achieved = algorithmic bytes / that,
                against 8 TB/s; traffic = FETCH_SIZE + WRITE_SIZE bytes per
                launch from the committed rocprofv3 summary, scaled by the
                same counters on a 1 GiB copy
  cpu_baseline  the oracle's NumPy paged_attention (the reference's kernel)
                on fp32 copies of a bounded sample of the same batch
  legs          the other synthetic workloads, each with absolute numbers and
                roofline fractions: mixed prefill+decode in one launch, the
                speculative-verify step with GPU greedy acceptance, the
                copy-on-write block copy, and the 48-request end-to-end mix
                (plus the shared-prefix mix) through HipRunner next to the
                NumPy runner on this host's cores.
Algorithmic bytes count each K/V element once and never the padding of a
partly filled block; flops count 4 * head_dim per unmasked (query, key) pair
and query head.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "vllm-lite_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "paged-attn HBM GB/s (% of peak) + e2e output tok/s on 48-req ragged mix"
PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "decode_256seq_traffic.md")


def events(torch, n):
    return [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(n)]


def median_ms(ev):
    return float(np.median([a.elapsed_time(b) for a, b in ev]))


def decode_leg(torch, ops, syn, steps, warmup, profile_only=False, layout="token"):
    """layout "head": the same cache as head-major blocks [blocks, Hkv, 16,
    D] (one KV head's 16 rows of a block are one 4 KB span)."""
    b = syn.build(torch, syn.decode_256_seqs(0))
    # this step's K/V are part of the cached context for the decode-only batch
    b["kc"][b["slot_mapping"].long()] = b["knew"]
    b["vc"][b["slot_mapping"].long()] = b["vnew"]
    kc, vc = b["kc"], b["vc"]
    if layout == "head":
        kc, vc = syn.to_head_major(kc, syn.BS), syn.to_head_major(vc, syn.BS)
    S = len(b["seqs"])
    out = torch.empty_like(b["q"])
    ws = ops.AttentionWorkspace().get(
        ops.paged_attention_workspace_size(S, S, syn.H, syn.D, int(b["ctx"].max())))
    ops.paged_attention_plan(b["q"], kc, b["seq_lens"], b["qsl"], syn.BS, ws)

    def step():
        ops.paged_attention_run(out, b["q"], kc, vc, b["bt"], b["seq_lens"], b["qsl"],
                                b["scale"], syn.BS, ws, max_query_len=1, min_query_len=1)

    def planned_step():
        ops.paged_attention_plan(b["q"], kc, b["seq_lens"], b["qsl"], syn.BS, ws)
        step()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # the launch's own duration: an event pair around each launch
    ev = events(torch, steps)
    for e0, e1 in ev:
        e0.record()
        step()
        e1.record()
    torch.cuda.synchronize()
    # a standalone step: the plan and the run, event pair around both
    ev_plan = events(torch, steps)
    for e0, e1 in ev_plan:
        e0.record()
        planned_step()
        e1.record()
    torch.cuda.synchronize()
    # the step rate: `steps` launches back to back, host clock around them
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    res = {"kernel_ms": median_ms(ev), "ms_per_step": wall * 1e3 / steps,
           "plan_and_run_ms": median_ms(ev_plan),
           "bytes": syn.algorithmic_bytes(b, with_scatter=False), "batch": b}
    if not profile_only:
        res["check_rel_err"] = syn.torch_reference_check(
            torch, b, out, np.linspace(0, S - 1, 8).astype(int))
    return res


def traffic_from_summary():
    """FETCH_SIZE + WRITE_SIZE bytes per decode launch (copy-calibrated) as
    recorded in the committed rocprofv3 summary, or None."""
    try:
        with open(TRAFFIC_SUMMARY) as f:
            m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", f.read())
        return int(m.group(1)) if m else None
    except OSError:
        return None


def cpu_baseline(torch, b, budget_s=12.0):
    """The oracle's per-sequence paged_attention (the reference's NumPy
    kernel) on fp32 copies of a bounded sample of the decode batch."""
    from oracle.attention import gather_slots, paged_attention
    try:
        from threadpoolctl import threadpool_info
        blas_threads = max([d.get("num_threads", 1) for d in threadpool_info()] or [1])
    except Exception:  # pragma: no cover
        blas_threads = 1
    cores = len(os.sched_getaffinity(0))
    S = len(b["seqs"])
    sample = list(range(0, S, 8))
    data = []
    for i in sample:
        nb = (int(b["ctx"][i]) + b["bs"] - 1) // b["bs"]
        slots = gather_slots(b["tables_np"][i, :nb], b["bs"], int(b["ctx"][i]))
        sl = torch.from_numpy(slots).cuda()
        data.append((b["q"][i:i + 1].float().cpu().numpy(), b["kc"][sl].float().cpu().numpy(),
                     b["vc"][sl].float().cpu().numpy(), np.arange(len(slots))))
    ctx = b["ctx"][sample]
    per_pass = int(ctx.sum()) * 2 * b["Hkv"] * b["D"] * 2 + 2 * len(sample) * b["H"] * b["D"] * 2

    def rate(budget):
        done_bytes, t0, reps = 0, time.perf_counter(), 0
        while True:
            for q, k, v, rs in data:
                paged_attention(q, k, v, rs, b["Hkv"], b["scale"])
            reps += 1
            done_bytes += per_pass
            if time.perf_counter() - t0 > budget or reps >= 50:
                break
        return done_bytes / (time.perf_counter() - t0) / 1e9, reps

    gbs, reps = rate(budget_s)
    one = None
    try:  # the same with one BLAS thread
        from threadpoolctl import threadpool_limits
        with threadpool_limits(limits=1):
            one = round(rate(budget_s / 2)[0], 3)
    except Exception:  # pragma: no cover
        pass
    return {"value": round(gbs, 3), "unit": "GB/s", "value_1_blas_thread": one,
            "cores": int(min(cores, blas_threads)), "kind": "port",
            "sample": f"{len(sample)} of {S} sequences (every 8th), {reps} passes of the oracle's "
                      f"NumPy paged_attention on fp32 copies, bytes counted at the bf16 size; "
                      f"{cores} visible cores, BLAS threads {blas_threads} (value_1_blas_thread: "
                      f"one BLAS thread, half the time budget)"}


def mixed_leg(torch, ops, syn, steps, warmup, profile_only=False, layout="token"):
    """Scatter + plan + one attention launch over 16 prefill chunks and 200
    decodes; also the prefill chunks alone and the decodes alone. profile_only
    names the one part to run (True: the mixed batch); layout "head": the
    caches as head-major blocks."""
    out = {}
    full = syn.mixed_8392_seqs(0)
    parts = {"mixed": full, "prefill_only": full[200:], "decode_only": full[:200]}
    for name, seqs in parts.items():
        if profile_only and name != (profile_only if isinstance(profile_only, str) else "mixed"):
            continue
        b = syn.build(torch, seqs, seed=2)
        S, T = len(seqs), int(b["q_lens"].sum())
        o = torch.empty_like(b["q"])
        ws = ops.AttentionWorkspace().get(
            ops.paged_attention_workspace_size(S, T, syn.H, syn.D, int(b["ctx"].max())))
        kc, vc = _layout_caches(syn, b, layout)

        def step():
            ops.reshape_and_cache(b["knew"], b["vnew"], kc, vc, b["slot_mapping"])
            ops.paged_attention_plan(b["q"], kc, b["seq_lens"], b["qsl"], syn.BS, ws)
            ops.paged_attention_run(o, b["q"], kc, vc, b["bt"], b["seq_lens"], b["qsl"],
                                    b["scale"], syn.BS, ws, max_query_len=b["max_q"],
                                    min_query_len=b["min_q"])

        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        ev = events(torch, steps)
        for e0, e1 in ev:
            e0.record()
            step()
            e1.record()
        torch.cuda.synchronize()
        ms = median_ms(ev)
        nbytes, flops = syn.algorithmic_bytes(b), syn.attention_flops(b)
        roof_ms = max(nbytes / (PEAK_HBM_GBS * 1e9), flops / (PEAK_BF16_TFLOPS * 1e12)) * 1e3
        r = {"us": round(ms * 1e3, 1), "tokens": T, "sequences": S, "sum_ctx": int(b["ctx"].sum()),
             "algorithmic_bytes": nbytes, "attention_flops": flops,
             "GBs": round(nbytes / ms / 1e6, 1), "hbm_frac": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4),
             "TFLOPs": round(flops / ms / 1e9, 1),
             "mfma_frac": round(flops / ms / 1e9 / PEAK_BF16_TFLOPS, 4),
             "roofline_us": round(roof_ms * 1e3, 1), "roofline_frac": round(roof_ms / ms, 4)}
        if not profile_only:
            _token_major_back(syn, b, kc, vc, layout)
            pick = [int(i) for i in np.linspace(0, S - 1, 6).astype(int)]
            r["check_rel_err"] = syn.torch_reference_check(torch, b, o, pick)
        out[name] = r
        del b, o, ws, kc, vc
        torch.cuda.empty_cache()
    out["workload"] = ("16 prefill chunks x 512 tokens with 0-2048 prior context + 200 decodes "
                       "with context 128-4096, H32/Hkv8/D128 bf16, block 16; a step = K/V scatter "
                       "of every new token + plan + one attention launch")
    return out


def _layout_caches(syn, b, layout):
    """The batch's caches for the timed steps: the token-major ones, or
    head-major copies."""
    if layout == "head":
        return syn.to_head_major(b["kc"], syn.BS), syn.to_head_major(b["vc"], syn.BS)
    return b["kc"], b["vc"]


def _token_major_back(syn, b, kc, vc, layout):
    """After head-major steps: the batch's token-major caches with what the
    steps scattered, for the reference check."""
    if layout == "head":
        b["kc"], b["vc"] = syn.to_token_major(kc), syn.to_token_major(vc)


def verify_leg(torch, ops, syn, steps, warmup, profile_only=False, layout="token"):
    """64 sequences x 5 query positions over contexts 1024..32768, then
    greedy acceptance of 4 drafts from fp32 logits [320, 32000]; layout
    "head": the caches as head-major blocks."""
    b = syn.build(torch, syn.verify_64x5_seqs(0), seed=3)
    kc, vc = _layout_caches(syn, b, layout)
    S, T = len(b["seqs"]), int(b["q_lens"].sum())
    V, K = 32000, 4
    o = torch.empty_like(b["q"])
    ws = ops.AttentionWorkspace().get(
        ops.paged_attention_workspace_size(S, T, syn.H, syn.D, int(b["ctx"].max())))
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    logits = torch.randn((T, V), generator=g, device="cuda")
    rng = np.random.default_rng(5)
    accept = rng.integers(0, K + 1, size=S)
    picks = torch.argmax(logits, dim=1).cpu().numpy()
    drafts = np.zeros((S, K), np.int32)
    for s in range(S):
        for r in range(K):
            p = int(picks[s * 5 + r])
            drafts[s, r] = p if r < accept[s] else (p + 1) % V
    row_start = torch.arange(0, T, 5, dtype=torch.int32, device="cuda")
    nd = torch.full((S,), K, dtype=torch.int32, device="cuda")
    dr = torch.from_numpy(drafts).cuda()
    toks = torch.empty((S, K + 1), dtype=torch.int32, device="cuda")
    nacc = torch.empty((S,), dtype=torch.int32, device="cuda")

    def step():
        ops.reshape_and_cache(b["knew"], b["vnew"], kc, vc, b["slot_mapping"])
        ops.paged_attention_plan(b["q"], kc, b["seq_lens"], b["qsl"], syn.BS, ws)
        ops.paged_attention_run(o, b["q"], kc, vc, b["bt"], b["seq_lens"], b["qsl"],
                                b["scale"], syn.BS, ws, max_query_len=5, min_query_len=5)
        ops.greedy_verify(logits, row_start, nd, dr, toks, nacc)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev = events(torch, steps)
    for e0, e1 in ev:
        e0.record()
        step()
        e1.record()
    torch.cuda.synchronize()
    ms = median_ms(ev)
    nbytes = syn.algorithmic_bytes(b) + T * V * 4 + S * (K + 2) * 4 * 2
    flops = syn.attention_flops(b)
    r = {"us": round(ms * 1e3, 1), "sum_ctx": int(b["ctx"].sum()), "algorithmic_bytes": nbytes,
         "attention_flops": flops, "GBs": round(nbytes / ms / 1e6, 1),
         "hbm_frac": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4),
         "workload": "64 sequences x 5 query positions (4 n-gram drafts + 1), context 1024-32768 "
                     "uniform, H32/Hkv8/D128 bf16, block 16; a step = scatter + plan + attention "
                     "+ greedy acceptance on logits [320, 32000] fp32"}
    if not profile_only:
        got_acc = nacc.cpu().numpy()
        got_tok = toks.cpu().numpy()
        ok = bool((got_acc == accept).all())
        for s in range(S):
            want = [int(picks[s * 5 + r]) for r in range(accept[s] + 1)]
            ok = ok and got_tok[s, :len(want)].tolist() == want and bool((got_tok[s, len(want):] == -1).all())
        r["acceptance_exact"] = ok
        _token_major_back(syn, b, kc, vc, layout)
        r["check_rel_err"] = syn.torch_reference_check(torch, b, o, [0, 21, 42, 63])
    del b, o, ws, logits, kc, vc
    torch.cuda.empty_cache()
    return r


def cow_leg(torch, ops, steps, warmup):
    """Copy-on-write of 48 partially filled shared tail blocks across the 6
    layers of the TinyLlama fp32 cache (K and V); the copies rotate over 8
    caches (600 MB) so that the 14 MB copied is not served from the
    Infinity Cache."""
    L, slots, hkv, hd, bs = 6, 512 * 16, 4, 48, 16
    caches = [(torch.randn((L, slots, hkv, hd), device="cuda"),
               torch.randn((L, slots, hkv, hd), device="cuda")) for _ in range(8)]
    rng = np.random.default_rng(6)
    src = rng.integers(0, 256, size=48)
    dst = 256 + rng.permutation(256)[:48]
    pairs = torch.from_numpy(np.stack([src, dst], 1).astype(np.int32)).cuda()
    for _ in range(warmup):
        ops.copy_blocks(*caches[0], pairs, bs)
    torch.cuda.synchronize()
    # back to back: `steps` launches between one event pair, each on the next
    # cache (as in a step, where the copy launch follows others on the stream)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for n in range(steps):
        ops.copy_blocks(*caches[n % 8], pairs, bs)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # one launch alone between its own event pair: adds the launch's fixed cost
    ev = events(torch, steps)
    for n, (a, b) in enumerate(ev):
        kc, vc = caches[n % 8]
        a.record()
        ops.copy_blocks(kc, vc, pairs, bs)
        b.record()
    torch.cuda.synchronize()
    ms_single = median_ms(ev)
    nbytes = 48 * L * bs * hkv * hd * 4 * 2 * 2
    ok = True
    for kc, vc in caches:  # every cache has been copied at least once
        for c in (kc, vc):
            blk = c.view(L, slots // bs, bs, hkv, hd)
            ok = ok and bool(torch.equal(blk[:, torch.from_numpy(dst).cuda().long()],
                                         blk[:, torch.from_numpy(src).cuda().long()]))
    del caches
    torch.cuda.empty_cache()
    return {"us": round(ms * 1e3, 2),
            "us_is": f"mean of {steps} back-to-back launches between one event pair",
            "us_single_launch": round(ms_single * 1e3, 2),
            "algorithmic_bytes": nbytes,
            "GBs": round(nbytes / ms / 1e6, 1), "hbm_frac": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4),
            "bit_exact": ok,
            "workload": "48 (src, dst) block pairs x 6 layers x K and V, TinyLlama cache "
                        "[6, 8192 slots, 4, 48] fp32, block 16"}


def engine_config(prefix_cache=False):
    """The 48-request mix's engine: TinyLlama 6 layers, d 384, H8/Hkv4, d_ff 1024,
    vocab 261, max_len 512; 512 blocks of 16; 16 seqs, budget 1024."""
    from vllmlite_amd.config import CacheConfig, EngineConfig, ModelConfig, SchedulerConfig
    return EngineConfig(
        model=ModelConfig(n_layers=6, n_heads=8, n_kv_heads=4, d_model=384, d_ff=1024,
                          vocab_size=261, max_seq_len=512),
        cache=CacheConfig(block_size=16, num_blocks=512, enable_prefix_caching=prefix_cache),
        scheduler=SchedulerConfig(max_seqs=16, max_batched_tokens=1024))


MIXES = {
    # name: (shared prefix tokens, fork every request after its first token)
    "mixed": (0, False),
    "shared_prefix": (256, False),
    "shared_prefix_forked": (256, True),
    "mixed_bf16_kv": (0, False),  # the 48-request mix over a bf16 K/V cache
    "mixed_head_major": (0, False),  # ... over head-major cache blocks
    "mixed_fp8_kv": (0, False),  # ... over an FP8 E4M3 K/V cache
}


def mix_config(name):
    from vllmlite_amd.workload import shared_prefix_config
    if name.startswith("mixed"):
        cfg = engine_config(False)
        if name == "mixed_bf16_kv":
            cfg.cache.kv_dtype = "bfloat16"
        if name == "mixed_head_major":
            cfg.cache.kv_layout = "head"
        if name == "mixed_fp8_kv":
            cfg.cache.kv_dtype = "float8_e4m3"
        return cfg
    return shared_prefix_config(True)


def run_mix(runner, cfg, name):
    """One pass of a mix: wall from the first add_request until drained (the
    reference's run_paged, bench/bench.py:74-109). Returns (wall, output
    tokens, steps, streams, copy-on-write pairs)."""
    from vllmlite_amd.engine import LLMEngine
    from vllmlite_amd.workload import drive_forked, mixed_lengths
    shared, fork = MIXES[name]
    counter = _CowCounter(runner) if fork else runner
    eng = LLMEngine(cfg, runner=counter)
    reqs = mixed_lengths(0, 48, shared)
    t0 = time.perf_counter()
    if fork:
        drive_forked(eng, reqs)
    else:
        for rid, ids, p in reqs:
            eng.add_request(params=p, request_id=rid, prompt_token_ids=ids)
        while eng.has_work:
            eng.step()
    wall = time.perf_counter() - t0
    streams = {rid: eng.seqs[rid].output_token_ids for rid in eng.seqs}
    return wall, eng.total_output_tokens, eng.total_steps, streams, counter.pairs if fork else 0


class _ZeroRunner:
    """A runner that computes nothing (zero logits): with greedy, ignore_eos
    requests the schedule does not depend on the tokens, so it replays the
    mix's batches for mix_floor."""

    def __init__(self, vocab):
        self.vocab_size = vocab
        self.batches = []

    def execute(self, out):
        rows, R = [], 0
        for item in out.scheduled:
            c = min(1 + len(item.seq.draft_token_ids), item.num_tokens)
            rows.append((R, c))
            R += c
        self.batches.append([(item.start_pos, item.num_tokens) for item in out.scheduled])
        return np.zeros((R, self.vocab_size), np.float32), rows


def mix_floor(cfg, name):
    """The device floor of a mix at 8 TB/s: per step, every weight once (the
    layers' projections and norms, lm_head, the embedding rows of the step's
    tokens) plus every K/V element the step's attention reads (each
    sequence's context, all layers) and writes (its new tokens), summed over
    the mix's steps."""
    from vllmlite_amd.engine import LLMEngine
    from vllmlite_amd.workload import drive_forked, mixed_lengths
    mc = cfg.model
    shared, fork = MIXES[name]
    zr = _ZeroRunner(mc.vocab_size)
    eng = LLMEngine(cfg, runner=zr)
    reqs = mixed_lengths(0, 48, shared)
    if fork:
        drive_forked(eng, reqs)
    else:
        for rid, ids, p in reqs:
            eng.add_request(params=p, request_id=rid, prompt_token_ids=ids)
        while eng.has_work:
            eng.step()
    d, hd, f = mc.d_model, mc.head_dim, mc.d_ff
    per_layer = (d * (mc.n_heads + 2 * mc.n_kv_heads) * hd + mc.n_heads * hd * d
                 + 2 * d * f + f * d + 2 * d) * 4
    weights = mc.n_layers * per_layer + (d * mc.vocab_size + d) * 4
    es = {"bfloat16": 2, "float8_e4m3": 1}.get(cfg.cache.kv_dtype, 4)
    row = mc.n_kv_heads * hd * es * 2 * mc.n_layers  # K and V of one token, every layer
    total = 0
    for b in zr.batches:
        toks = sum(n for _, n in b)
        total += weights + toks * d * 4 + sum((st + n) * row + n * row for st, n in b)
    return {"steps": len(zr.batches), "bytes_per_step": round(total / len(zr.batches)),
            "floor_us_per_step": round(total / len(zr.batches) / PEAK_HBM_GBS / 1e3, 2)}


class _CowCounter:
    """A runner wrapper that counts the copy-on-write pairs it is handed."""

    def __init__(self, runner):
        self.runner = runner
        self.pairs = 0
        self.vocab_size = runner.vocab_size
        if hasattr(runner, "execute_argmax"):
            self.execute_argmax = self._argmax

    def execute(self, out):
        self.pairs += len(out.cow)
        return self.runner.execute(out)

    def _argmax(self, out):
        self.pairs += len(out.cow)
        return self.runner.execute_argmax(out)


def mc_layers(cfg):
    return cfg.model.n_layers


def launch_floor_us(n, reps=50):
    """The time per replay of a HIP graph of n dependent launches that each
    copy one int32 word with one workgroup (the least a launch does), replayed
    back to back: the floor, on this GPU, of a step made of n dependent
    launches, whatever the kernels compute."""
    import torch
    from vllmlite_amd import ops
    a = torch.zeros(1, dtype=torch.int32, device="cuda")
    b = torch.zeros_like(a)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for i in range(n):
            ops.copy_words(b if i % 2 else a, a if i % 2 else b)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(n):
                ops.copy_words(b if i % 2 else a, a if i % 2 else b)
        g.replay()
        s.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            g.replay()
        e1.record(s)
        e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def e2e_leg(name="mixed", repeat=3, cpu=True):
    """Output tok/s of a mix through HipRunner (one warm-up pass, then best of
    `repeat`; the runner and its captured graphs persist across passes, each
    pass gets a fresh engine), the streams checked against the reference's,
    and the same mix through the NumPy oracle runner on this host's cores
    (warm-up on a 4-request mix, best of `repeat`)."""
    from vllmlite_amd.hip_runner import HipRunner
    cfg = mix_config(name)
    runner = HipRunner(cfg.model, cfg.cache)
    run_mix(runner, cfg, name)
    wall, toks, steps, streams, pairs = min(
        (run_mix(runner, cfg, name) for _ in range(repeat)), key=lambda r: r[0])
    shared, fork = MIXES[name]
    out = {"workload": ("48-request ragged mix" +
                        (f" behind a {shared}-token shared prefix, prefix cache on" if shared
                         else "") +
                        (", every request forked once after its first token (copy-on-write of "
                         "its partial shared tail)" if fork else "") +
                        f" (greedy), TinyLlama 6L d384 H8/Hkv4 d_ff1024 fp32"
                        f"{', bf16 K/V cache' if cfg.cache.kv_dtype == 'bfloat16' else ''}"
                        f"{', FP8 E4M3 K/V cache' if cfg.cache.kv_dtype == 'float8_e4m3' else ''}"
                        f"{', head-major cache blocks' if cfg.cache.kv_layout == 'head' else ''}, "
                        "block 16, "
                        f"{cfg.cache.num_blocks} blocks, max_len {cfg.model.max_seq_len}, "
                        "16 seqs, budget 1024"),
           "output_tok_per_s": round(toks / wall, 1), "wall_s": round(wall, 4),
           "steps": steps, "us_per_step": round(wall / steps * 1e6, 1), "output_tokens": toks}
    fl = mix_floor(cfg, name)
    n_launch = mc_layers(cfg) * (4 if runner._fused_wo else 5) + 1
    lf = launch_floor_us(n_launch)
    out["roofline"] = {
        "bound": "hbm (weights + K/V per step at 8 TB/s; the steps are launch- and "
                 "latency-bound far above it)",
        "floor_us_per_step": fl["floor_us_per_step"], "bytes_per_step": fl["bytes_per_step"],
        "frac": round(fl["floor_us_per_step"] / (wall / steps * 1e6), 4),
        "device_launches_per_decode_step": n_launch,
        "launch_floor_us_per_step": round(lf, 1),
        "launch_floor_frac": round(lf / (wall / steps * 1e6), 4),
        "launch_floor_is": ("a graph of that many dependent one-workgroup launches (each copying "
                            "one word) replayed back to back on this GPU: the floor of the "
                            "decode step's launch structure, whatever the kernels compute"),
        "launches_are": ("per layer QKV+RoPE+scatter (layer 0 also gathers the embeddings, "
                         "resolves the previous step's ids, reads its indices from the step's "
                         "pinned record and copies the record to the device), attention"
                         + (" with wo (one partial row per KV head), residual+norm+gate|up+SwiGLU"
                            if runner._fused_wo else ", wo+residual, norm+gate|up+SwiGLU")
                         + ", down+residual; then lm_head with each row's argmax")}
    if fork:
        out["cow_pairs"] = pairs
    fixture, key = (("cfg0_streams.json", None) if name.startswith("mixed") else
                    ("shared_prefix_streams.json", "forked" if fork else "plain"))
    with open(os.path.join(ROOT, "tests", "golden", fixture)) as f:
        gold = json.load(f)
    gold = gold["streams"] if key is None else gold[key]["streams"]
    same = sum(streams.get(r) == gold[r] for r in gold)
    out["streams_identical_to_reference"] = f"{same}/{len(gold)}"
    if cfg.cache.kv_dtype != "float32":
        out["streams_note"] = ("the reference caches fp32; against the oracle runner with the "
                               "same narrow cache the streams are checked by the GPU tests")
    if cpu:
        from oracle.runner import NumpyRunner
        from vllmlite_amd.engine import LLMEngine
        from vllmlite_amd.workload import make_workload
        warm = make_workload(4, np.random.default_rng(99), 16, 64, 8, 16)
        eng = LLMEngine(cfg, runner=NumpyRunner(cfg.model, cfg.cache))
        for rid, ids, p in warm:
            eng.add_request(params=p, request_id=rid, prompt_token_ids=ids)
        while eng.has_work:
            eng.step()
        cpu_best = min((run_mix(NumpyRunner(cfg.model, cfg.cache), cfg, name)
                        for _ in range(repeat)), key=lambda r: r[0])
        cpu_tps = cpu_best[1] / cpu_best[0]
        out["cpu_numpy_tok_per_s"] = round(cpu_tps, 1)
        out["cpu_cores"] = len(os.sched_getaffinity(0))
        out["speedup_vs_cpu_numpy"] = round(toks / wall / cpu_tps, 2)
        out["cpu_streams_identical"] = cpu_best[3] == streams
        try:  # one pass with one BLAS thread
            from threadpoolctl import threadpool_limits
            with threadpool_limits(limits=1):
                one = run_mix(NumpyRunner(cfg.model, cfg.cache), cfg, name)
            out["cpu_numpy_tok_per_s_1_blas_thread"] = round(one[1] / one[0], 1)
            out["speedup_vs_cpu_numpy_1_blas_thread"] = round(toks / wall / (one[1] / one[0]), 2)
        except Exception:  # pragma: no cover
            pass
    return out


def copy_ceiling(torch, nbytes=2 << 30, iters=10):
    a = torch.empty(nbytes // 2, dtype=torch.bfloat16, device="cuda")
    c = torch.empty_like(a)
    c.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        c.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / iters
    return 2 * nbytes / (ms * 1e-3) / 1e9


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end mixes")
    ap.add_argument("--legs", default="decode,mixed,verify,cow,e2e",
                    help="comma-separated legs to run (decode is always run)")
    ap.add_argument("--profile-mode", default=None, metavar="LEG",
                    help="only the timed launches of one leg (decode, mixed, prefill, verify, cow, "
                         "e2e), for rocprofv3 passes")
    ap.add_argument("--copy-only", action="store_true",
                    help="only 5 device copies of 1 GiB (calibrates rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE against a kernel of known traffic)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the attention step runs on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured configuration)", file=sys.stderr)
        sys.exit(2)

    import torch
    from vllmlite_amd import ops
    from vllmlite_amd import synthetic as syn

    torch.cuda.set_device(0)
    if args.copy_only:
        a = torch.ones(1 << 29, dtype=torch.bfloat16, device="cuda")
        c = torch.empty_like(a)
        for _ in range(5):
            c.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_only": True, "bytes_read_per_copy": a.numel() * 2,
                          "bytes_written_per_copy": c.numel() * 2}), flush=True)
        return
    if args.profile_mode:
        leg = args.profile_mode
        fn = {"decode": lambda: decode_leg(torch, ops, syn, args.steps, args.warmup, True),
              "mixed": lambda: mixed_leg(torch, ops, syn, args.steps, args.warmup, True),
              "prefill": lambda: mixed_leg(torch, ops, syn, args.steps, args.warmup,
                                           "prefill_only"),
              "verify": lambda: verify_leg(torch, ops, syn, args.steps, args.warmup, True),
              "cow": lambda: cow_leg(torch, ops, args.steps, args.warmup),
              "e2e": lambda: e2e_leg("mixed", cpu=False)}[leg]
        r = fn()
        r.pop("batch", None)
        print(json.dumps({"profile_mode": leg, "result": r}), flush=True)
        return

    legs = set(args.legs.split(","))
    d = decode_leg(torch, ops, syn, args.steps, args.warmup)
    b = d.pop("batch")
    nbytes = d["bytes"]
    achieved = nbytes / (d["kernel_ms"] * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(nbytes / (d["ms_per_step"] * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 Q/K/V, NaN-poisoned unowned blocks)",
        "config": {"workload": "ragged decode paged attention, 256 seqs x 1 query, ctx lognormal "
                               "median 1024 sigma 0.6 clipped 64-8192, H32/Hkv8/D128, block 16, "
                               "2^17-block pool",
                   "sum_ctx": int(b["ctx"].sum()), "algorithmic_bytes": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": traffic_from_summary()},
        "kernel_us": round(d["kernel_ms"] * 1e3, 2),
        "kernel_us_is": "median of per-launch HIP event pairs (the run launch; the plan is "
                        "built once per step for all layers and timed below)",
        "plan_and_run_us": round(d["plan_and_run_ms"] * 1e3, 2),
        "plan_and_run_hbm_frac": round(nbytes / (d["plan_and_run_ms"] * 1e-3) / 1e9
                                       / PEAK_HBM_GBS, 4),
        "check_rel_err": d["check_rel_err"],
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(torch, b)
    del b
    torch.cuda.empty_cache()
    line["copy_ceiling_gbs"] = round(copy_ceiling(torch), 1)
    extra = {}
    # the same batch over head-major cache blocks [blocks, Hkv, 16, D]
    h = decode_leg(torch, ops, syn, args.steps, args.warmup, layout="head")
    h.pop("batch")
    extra["decode_head_major"] = {
        "kernel_us": round(h["kernel_ms"] * 1e3, 2),
        "hbm_frac": round(nbytes / (h["kernel_ms"] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        "ms_per_step": round(h["ms_per_step"], 4), "check_rel_err": h["check_rel_err"],
        "layout": "head-major blocks [blocks, Hkv, 16, D]: a KV head's 16 rows are one 4 KB span"}
    del h
    torch.cuda.empty_cache()
    if "mixed" in legs:
        extra["mixed_prefill_decode"] = mixed_leg(torch, ops, syn, 20, 3)
    if "verify" in legs:
        extra["spec_verify"] = verify_leg(torch, ops, syn, 20, 3)
    if "cow" in legs:
        extra["copy_on_write"] = cow_leg(torch, ops, 50, 5)
    if "e2e" in legs and not args.no_e2e:
        line["e2e"] = e2e_leg("mixed", cpu=not args.no_cpu)
        extra["e2e_shared_prefix"] = e2e_leg("shared_prefix", cpu=not args.no_cpu)
        extra["e2e_shared_prefix_forked"] = e2e_leg("shared_prefix_forked", cpu=False)
        extra["e2e_bf16_kv_cache"] = e2e_leg("mixed_bf16_kv", cpu=False)
        extra["e2e_head_major_cache"] = e2e_leg("mixed_head_major", cpu=False)
        extra["e2e_fp8_kv_cache"] = e2e_leg("mixed_fp8_kv", cpu=False)
    line["legs"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

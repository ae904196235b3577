#!/usr/bin/env python3
"""Benchmark of the ragged paged-attention step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--profile-mode]

The timed workload is the 256-sequence ragged decode batch: 256 sequences of
one query token, context lengths lognormal (median 1024, sigma 0.6) clipped
to 64..8192, 32 query heads over 8 KV heads, head_dim 128, bf16 Q/K/V
~N(0,1), block size 16, block tables drawn as consecutive slices of a seeded
permutation of a 2^17-block pool (8.6 GB of K/V; every block a sequence does
not own is NaN). A step is one paged-attention run over that batch with the
inputs already resident in HBM; the work plan is built once outside the timed
region, as the runner does once per step for all layers.

The JSON line reports:
  value         algorithmic HBM bytes per step / measured step time (GB/s)
  roofline      the attention kernel's average duration from HIP events on
                torch's stream, algorithmic bytes / that, against 8 TB/s
  cpu_baseline  the NumPy oracle (the reference's per-sequence paged_attention
                on fp32 copies of the same bf16 data), timed on this host
Algorithmic bytes = sum(ctx) * 2 (K,V) * 8 heads * 128 * 2 B + Q read + out
write (256 * 32 * 128 * 2 B each) + block-table entries read (4 B per block)
+ seq_lens (4 B per sequence): each K/V element once, no block padding.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "vllm-lite_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "paged-attn HBM GB/s (% of peak) + e2e output tok/s on 48-req ragged mix"
PEAK_HBM_GBS = 8000.0
S, H, HKV, D, BS, POOL = 256, 32, 8, 128, 16, 1 << 17
SIGMA = 0.6


def decode_lengths(seed=0, n=S, sigma=SIGMA):
    rng = np.random.default_rng(seed)
    ctx = np.clip(np.rint(rng.lognormal(np.log(1024.0), sigma, size=n)), 64, 8192).astype(np.int64)
    return ctx, rng


def algorithmic_bytes(ctx):
    nblk = (ctx + BS - 1) // BS
    return int(ctx.sum() * 2 * HKV * D * 2 + 2 * len(ctx) * H * D * 2 + nblk.sum() * 4 + 4 * len(ctx))


def build_decode_batch(torch, seed=0):
    """Device tensors of the 256-sequence batch; returns a dict."""
    ctx, rng = decode_lengths(seed)
    nblk = (ctx + BS - 1) // BS
    perm = rng.permutation(POOL).astype(np.int64)
    W = int(nblk.max())
    tables = np.zeros((S, W), np.int32)
    off = 0
    owned = []
    for i in range(S):
        t = perm[off:off + nblk[i]]
        off += nblk[i]
        tables[i, :nblk[i]] = t
        owned.append((t[:, None] * BS + np.arange(BS)[None, :]).reshape(-1)[:ctx[i]])
    slots = torch.from_numpy(np.concatenate(owned)).cuda()
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    dev = "cuda"
    kc = torch.full((POOL * BS, HKV, D), float("nan"), dtype=torch.bfloat16, device=dev)
    vc = torch.full((POOL * BS, HKV, D), float("nan"), dtype=torch.bfloat16, device=dev)
    n = slots.numel()
    kc[slots] = torch.randn((n, HKV, D), generator=g, device=dev).to(torch.bfloat16)
    vc[slots] = torch.randn((n, HKV, D), generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn((S, H, D), generator=g, device=dev).to(torch.bfloat16)
    qsl = torch.arange(S + 1, dtype=torch.int32, device=dev)
    return dict(ctx=ctx, tables_np=tables, q=q, kc=kc, vc=vc,
                bt=torch.from_numpy(tables).cuda(), seq_lens=torch.from_numpy(ctx.astype(np.int32)).cuda(),
                qsl=qsl, scale=1.0 / np.sqrt(D))


def spot_check(torch, b, out, n_check=6):
    """A few sequences against the oracle on fp32 copies (not timed)."""
    from oracle.attention import gather_slots, paged_attention
    idx = np.linspace(0, S - 1, n_check).astype(int)
    worst = 0.0
    for i in idx:
        t = b["tables_np"][i, :(b["ctx"][i] + BS - 1) // BS]
        slots = gather_slots(t, BS, int(b["ctx"][i]))
        sl = torch.from_numpy(slots).cuda()
        k = b["kc"][sl].float().cpu().numpy()
        v = b["vc"][sl].float().cpu().numpy()
        q = b["q"][i:i + 1].float().cpu().numpy()
        want = paged_attention(q, k, v, np.arange(len(slots)), HKV, b["scale"])
        got = out[i:i + 1].float().cpu().numpy()
        err = np.abs(got - want).max() / max(1e-6, np.abs(want).max())
        worst = max(worst, float(err))
    return worst


def cpu_baseline(torch, b, budget_s=12.0):
    """The oracle's per-sequence paged_attention (the reference's NumPy
    kernel) on fp32 copies of a bounded sample of the sequences."""
    from oracle.attention import gather_slots, paged_attention
    try:
        from threadpoolctl import threadpool_info
        blas_threads = max([d.get("num_threads", 1) for d in threadpool_info()] or [1])
    except Exception:  # pragma: no cover
        blas_threads = 1
    cores = len(os.sched_getaffinity(0))
    # compact copy of a sample of sequences (every 8th), fp32
    sample = list(range(0, S, 8))
    data = []
    for i in sample:
        t = b["tables_np"][i, :(b["ctx"][i] + BS - 1) // BS]
        slots = gather_slots(t, BS, int(b["ctx"][i]))
        sl = torch.from_numpy(slots).cuda()
        data.append((b["q"][i:i + 1].float().cpu().numpy(), b["kc"][sl].float().cpu().numpy(),
                     b["vc"][sl].float().cpu().numpy(), np.arange(len(slots))))
    done_bytes, t0, reps = 0, time.perf_counter(), 0
    while True:
        for (q, k, v, rs), i in zip(data, sample):
            paged_attention(q, k, v, rs, HKV, b["scale"])
        reps += 1
        done_bytes += algorithmic_bytes(b["ctx"][sample])
        if time.perf_counter() - t0 > budget_s or reps >= 50:
            break
    dt = time.perf_counter() - t0
    return {"value": round(done_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": int(min(cores, blas_threads)),
            "kind": "port",
            "sample": f"{len(sample)} of {S} sequences (every 8th), {reps} passes, fp32 NumPy, "
                      f"bytes counted at the bf16 workload size; {cores} visible cores, "
                      f"BLAS threads {blas_threads}"}


def cfg0_engine_config():
    """The 48-request mix's engine: TinyLlama 6 layers, d 384, H8/Hkv4, d_ff 1024,
    vocab 261, max_len 512; 512 blocks of 16, no prefix cache; 16 seqs, budget 1024."""
    from vllmlite_amd.config import CacheConfig, EngineConfig, ModelConfig, SchedulerConfig
    return EngineConfig(
        model=ModelConfig(n_layers=6, n_heads=8, n_kv_heads=4, d_model=384, d_ff=1024,
                          vocab_size=261, max_seq_len=512),
        cache=CacheConfig(block_size=16, num_blocks=512, enable_prefix_caching=False),
        scheduler=SchedulerConfig(max_seqs=16, max_batched_tokens=1024))


def run_mix(runner, cfg):
    """One pass of the mix: wall from the first add_request until drained
    (the reference's run_paged, bench/bench.py:74-109)."""
    from vllmlite_amd.engine import LLMEngine
    from vllmlite_amd.workload import mixed_lengths
    eng = LLMEngine(cfg, runner=runner)
    reqs = mixed_lengths(0, 48, 0)
    t0 = time.perf_counter()
    for rid, ids, p in reqs:
        eng.add_request(params=p, request_id=rid, prompt_token_ids=ids)
    while eng.has_work:
        eng.step()
    wall = time.perf_counter() - t0
    streams = {rid: list(eng.seqs[rid].output_token_ids) for rid, _, _ in reqs}
    return wall, eng.total_output_tokens, eng.total_steps, streams


def e2e_leg(repeat=3, cpu=True):
    """Output tok/s of the 48-request mix through HipRunner (one warm-up pass,
    then best of `repeat`; the runner and its captured graphs persist across
    passes, each pass gets a fresh engine), and the same mix through the NumPy
    oracle runner on this host's cores (warm-up on a 4-request mix, best of
    `repeat`)."""
    import json as _json
    from vllmlite_amd.hip_runner import HipRunner
    cfg = cfg0_engine_config()
    runner = HipRunner(cfg.model, cfg.cache)
    run_mix(runner, cfg)
    best = min((run_mix(runner, cfg) for _ in range(repeat)), key=lambda r: r[0])
    wall, toks, steps, streams = best
    with open(os.path.join(ROOT, "tests", "golden", "cfg0_streams.json")) as f:
        gold = _json.load(f)["streams"]
    same = sum(streams[r] == gold[r] for r in gold)
    out = {"workload": "48-request ragged mix (prompts 17-251, outputs 16-192, greedy), "
                       "TinyLlama 6L d384 H8/Hkv4 d_ff1024 fp32, block 16, 512 blocks, "
                       "16 seqs, budget 1024",
           "output_tok_per_s": round(toks / wall, 1), "wall_s": round(wall, 4),
           "steps": steps, "us_per_step": round(wall / steps * 1e6, 1),
           "output_tokens": toks, "streams_identical_to_reference": f"{same}/{len(gold)}"}
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
        cpu_best = min((run_mix(NumpyRunner(cfg.model, cfg.cache), cfg) for _ in range(repeat)),
                       key=lambda r: r[0])
        cpu_tps = cpu_best[1] / cpu_best[0]
        out["cpu_numpy_tok_per_s"] = round(cpu_tps, 1)
        out["cpu_cores"] = len(os.sched_getaffinity(0))
        out["speedup_vs_cpu_numpy"] = round(toks / wall / cpu_tps, 2)
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
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-e2e", action="store_true", help="skip the 48-request mix leg")
    ap.add_argument("--e2e-only", action="store_true",
                    help="only the 48-request mix through HipRunner (for rocprofv3 passes)")
    ap.add_argument("--profile-mode", action="store_true",
                    help="only the timed attention runs (for rocprofv3 passes)")
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
    if args.e2e_only:
        print(json.dumps({"e2e": e2e_leg(cpu=False)}), flush=True)
        return
    b = build_decode_batch(torch)
    nbytes = algorithmic_bytes(b["ctx"])
    out = torch.empty_like(b["q"])
    ws = ops.AttentionWorkspace().get(
        ops.paged_attention_workspace_size(S, S, H, D, int(b["ctx"].max())))
    ops.paged_attention_plan(b["q"], b["kc"], b["seq_lens"], b["qsl"], BS, ws)

    def step():
        ops.paged_attention_run(out, b["q"], b["kc"], b["vc"], b["bt"], b["seq_lens"], b["qsl"],
                                b["scale"], BS, ws, max_query_len=1)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e0, e1 in ev:
        e0.record()
        step()
        e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kernel_ms = float(np.mean([e0.elapsed_time(e1) for e0, e1 in ev]))
    ms_per_step = wall * 1e3 / args.steps
    if args.profile_mode:
        print(json.dumps({"profile_mode": True, "kernel_ms": kernel_ms}))
        return

    rel_err = spot_check(torch, b, out)
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(nbytes / (ms_per_step * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
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
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None},
        "kernel_us": round(kernel_ms * 1e3, 2),
        "copy_ceiling_gbs": round(copy_ceiling(torch), 1),
        "spot_check_max_rel_err": rel_err,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(torch, b)
    del b, out, ws
    torch.cuda.empty_cache()
    if not args.no_e2e:
        line["e2e"] = e2e_leg(cpu=not args.no_cpu)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

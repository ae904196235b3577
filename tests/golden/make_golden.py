"""Writes the golden fixtures that only the reference itself can pin.

Run in the build container (where the reference is mounted read-only at
/root/reference), never on a GPU machine:

    python tests/golden/make_golden.py

Outputs (small JSON, committed):
  cfg0_streams.json   per-request greedy output ids of the 48-request mix
                      (6 layers, d 384, H8/Hkv4, d_ff 1024, max_len 512,
                      block 16, 512 blocks, max_seqs 16, budget 1024, seed 0)
                      plus the top-1 minus top-2 logit margin of each emitted
                      token, and the step count;
  weights_sha256.json sha256 of every weight tensor for that model config and
                      for the small invariance-test config;
  small_streams.json  greedy streams of the 4 invariance prompts on the small
                      engine (2 layers, d 64, H4/Hkv2, d_ff 128);
  shared_prefix_streams.json
                      the 48-request mix behind a 256-token shared system
                      prompt (bench/bench.py:35-47 with shared_prefix 256,
                      max_len 768, 768 blocks, prefix cache on): greedy
                      streams and step count ("plain"), and the same mix with
                      every request forked once, right after its first token,
                      through the reference's BlockManager.fork
                      (vllmlite/block_manager.py:133-137) so that the first
                      write into each shared partial tail block emits a
                      copy-on-write pair (block_manager.py:74-85): streams of
                      parents and children, step count, and the number of CoW
                      pairs with the prompt lengths whose tails were partial
                      ("forked").
  sampling_choices.json
                      seeded draws of the reference's sample()
                      (vllmlite/sampling.py:41-64) on rows of 64 logits taken
                      from a few values, so that ties are common, under a grid
                      of temperature / top_k / top_p / repetition penalty /
                      min_tokens settings: the row, the settings, the seed
                      and three successive draws from one generator.

`python tests/golden/make_golden.py sampling` writes only the last file.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REF)

from vllmlite.config import CacheConfig, EngineConfig, ModelConfig, SchedulerConfig  # noqa: E402
from vllmlite.engine import LLMEngine, _Detok  # noqa: E402
from vllmlite.model import Layer, TinyLlama  # noqa: E402
from vllmlite.sampling import sample  # noqa: E402
from vllmlite.sequence import SamplingParams, Sequence  # noqa: E402
from bench.bench import make_workload  # noqa: E402


def weight_hashes(mc):
    m = TinyLlama(mc, 16)
    out = {"tok_emb": hashlib.sha256(m.tok_emb.tobytes()).hexdigest(),
           "lm_head": hashlib.sha256(m.lm_head.tobytes()).hexdigest(),
           "final_norm": hashlib.sha256(m.final_norm.tobytes()).hexdigest()}
    for i, layer in enumerate(m.layers):
        for name in Layer.__slots__:
            out[f"layers.{i}.{name}"] = hashlib.sha256(getattr(layer, name).tobytes()).hexdigest()
    return out


def run_with_margins(engine, reqs):
    """Drive the engine; record each emitted token's top1-top2 logit margin."""
    margins = {rid: [] for rid, _, _ in reqs}
    real_execute = engine.runner.execute
    captured = {}

    def execute(sched):
        logits, rows = real_execute(sched)
        captured["sched"], captured["logits"], captured["rows"] = sched, logits, rows
        return logits, rows

    engine.runner.execute = execute
    for rid, ids, params in reqs:
        engine.add_request(params=params, request_id=rid, prompt_token_ids=ids)
    while engine.has_work:
        before = {rid: len(s.output_token_ids) for rid, s in engine.seqs.items()}
        engine.step()
        sched = captured.get("sched")
        if sched is None:
            continue
        for i, item in enumerate(sched.scheduled):
            seq = item.seq
            if len(seq.output_token_ids) > before[seq.request_id]:
                row0, count = captured["rows"][i]
                row = np.sort(captured["logits"][row0 + count - 1].astype(np.float64))
                margins[seq.request_id].append(float(row[-1] - row[-2]))
        captured.clear()
    return margins


def fork_child(engine, parent, child_id):
    """A running copy of `parent` that shares all of its blocks, partial tail
    included, made with the reference's own BlockManager.fork. The child
    joins the running list after its parent's peers; its stream continues
    from the parent's state."""
    child = Sequence(child_id, list(parent.prompt_token_ids), parent.params)
    child.output_token_ids = list(parent.output_token_ids)
    child.num_computed = parent.num_computed
    child.status = parent.status
    engine.scheduler.blocks.fork(parent, child)
    engine.scheduler.blocks.live_tokens += child.table.num_filled
    engine.scheduler.running.append(child)
    engine.seqs[child_id] = child
    engine.detok[child_id] = _Detok(engine.detok[parent.request_id].text,
                                    engine.detok[parent.request_id].consumed)
    engine.rngs[child_id] = np.random.default_rng(parent.params.seed)
    return child


def shared_prefix_runs():
    mc = ModelConfig(n_layers=6, n_heads=8, n_kv_heads=4, d_model=384, d_ff=1024,
                     vocab_size=261, max_seq_len=768)
    reqs = make_workload(48, np.random.default_rng(0), 16, 256, 16, 192, 256)
    out = {"prompts": {rid: [int(t) for t in ids] for rid, ids, _ in reqs},
           "max_tokens": {rid: int(p.max_tokens) for rid, _, p in reqs}}

    def engine():
        return LLMEngine(EngineConfig(
            model=mc, cache=CacheConfig(block_size=16, num_blocks=768, enable_prefix_caching=True),
            scheduler=SchedulerConfig(max_seqs=16, max_batched_tokens=1024)))

    eng = engine()
    for rid, ids, params in reqs:
        eng.add_request(params=params, request_id=rid, prompt_token_ids=ids)
    while eng.has_work:
        eng.step()
    st = eng.stats()
    out["plain"] = {"steps": eng.total_steps,
                    "output_tokens": eng.total_output_tokens,
                    "prefix_hit_rate": round(st["prefix_hit_rate"], 6),
                    "streams": {rid: [int(t) for t in eng.seqs[rid].output_token_ids]
                                for rid, _, _ in reqs}}

    eng = engine()
    pairs = []
    real_execute = eng.runner.execute

    def execute(sched):
        pairs.extend((int(a), int(b)) for a, b in sched.cow)
        return real_execute(sched)

    eng.runner.execute = execute
    for rid, ids, params in reqs:
        eng.add_request(params=params, request_id=rid, prompt_token_ids=ids)
    forked, partial = set(), []
    while eng.has_work:
        eng.step()
        for seq in list(eng.scheduler.running):
            rid = seq.request_id
            if rid in forked or rid.endswith(".c") or len(seq.output_token_ids) != 1:
                continue
            forked.add(rid)
            if seq.table.num_filled % 16:
                partial.append(rid)
            fork_child(eng, seq, rid + ".c")
    out["forked"] = {"steps": eng.total_steps,
                     "output_tokens": eng.total_output_tokens,
                     "cow_pairs": len(pairs),
                     "forked": sorted(forked, key=lambda r: int(r[1:])),
                     "partial_tails": partial,
                     "preemptions": eng.scheduler.total_preemptions,
                     "streams": {rid: [int(t) for t in s.output_token_ids]
                                 for rid, s in eng.seqs.items()}}
    return out


def sampling_cases():
    rng = np.random.default_rng(7)
    cases = []
    for temperature in (0.0, 0.7, 1.0, 1.3):
        for top_k in (0, 5, 20):
            for top_p in (1.0, 0.9, 0.5):
                for pen in (1.0, 1.3):
                    row = (rng.integers(-4, 5, 64) * 0.5).astype(np.float32)
                    seen = [int(t) for t in rng.integers(0, 64, 6)]
                    min_tokens = int(rng.integers(0, 3))
                    num_generated = int(rng.integers(0, 3))
                    seed = int(rng.integers(0, 2 ** 31))
                    params = SamplingParams(temperature=temperature, top_k=top_k, top_p=top_p,
                                            repetition_penalty=pen, min_tokens=min_tokens,
                                            seed=seed)
                    g = np.random.default_rng(seed)
                    draws = [sample(row, params, seen, g, num_generated, 2) for _ in range(3)]
                    cases.append({"row": [float(x) for x in row], "temperature": temperature,
                                  "top_k": top_k, "top_p": top_p, "repetition_penalty": pen,
                                  "min_tokens": min_tokens, "num_generated": num_generated,
                                  "eos_id": 2, "seen": seen, "seed": seed,
                                  "draws": [int(t) for t in draws]})
    return cases


def main():
    if sys.argv[1:] == ["sampling"]:
        with open(os.path.join(HERE, "sampling_choices.json"), "w") as f:
            json.dump({"cases": sampling_cases()}, f)
        return
    mc = ModelConfig(n_layers=6, n_heads=8, n_kv_heads=4, d_model=384, d_ff=1024,
                     vocab_size=261, max_seq_len=512)
    cc = CacheConfig(block_size=16, num_blocks=512, enable_prefix_caching=False)
    sc = SchedulerConfig(max_seqs=16, max_batched_tokens=1024)
    reqs = make_workload(48, np.random.default_rng(0), 16, 256, 16, 192, 0)
    eng = LLMEngine(EngineConfig(model=mc, cache=cc, scheduler=sc))
    margins = run_with_margins(eng, reqs)
    streams = {rid: [int(t) for t in eng.seqs[rid].output_token_ids] for rid, _, _ in reqs}
    prompts = {rid: [int(t) for t in ids] for rid, ids, _ in reqs}
    with open(os.path.join(HERE, "cfg0_streams.json"), "w") as f:
        json.dump({"steps": eng.total_steps, "prompts": prompts, "streams": streams,
                   "margins": {k: [round(x, 6) for x in v] for k, v in margins.items()}}, f)

    small = ModelConfig(n_layers=2, n_heads=4, n_kv_heads=2, d_model=64, d_ff=128, max_seq_len=512)
    with open(os.path.join(HERE, "weights_sha256.json"), "w") as f:
        json.dump({"cfg0": weight_hashes(mc), "small": weight_hashes(small)}, f, indent=0)

    prompts4 = ["the quick brown fox jumps over", "a",
                "systems programming is mostly about memory and never about", "hello"]
    e2 = LLMEngine(EngineConfig(
        model=ModelConfig(n_layers=2, n_heads=4, n_kv_heads=2, d_model=64, d_ff=128, max_seq_len=512),
        cache=CacheConfig(block_size=16, num_blocks=512, enable_prefix_caching=False),
        scheduler=SchedulerConfig(max_seqs=8, max_batched_tokens=1024)))
    p = SamplingParams(max_tokens=20, temperature=0.0, ignore_eos=True)
    ids = [e2.add_request(x, p) for x in prompts4]
    while e2.has_work:
        e2.step()
    with open(os.path.join(HERE, "small_streams.json"), "w") as f:
        json.dump({"prompts": prompts4, "max_tokens": 20,
                   "streams": [e2.seqs[i].output_token_ids for i in ids]}, f)
    sp = shared_prefix_runs()
    with open(os.path.join(HERE, "shared_prefix_streams.json"), "w") as f:
        json.dump(sp, f)
    print("shared prefix: plain", sp["plain"]["steps"], "steps,", sp["plain"]["output_tokens"],
          "tokens; forked", sp["forked"]["steps"], "steps,", sp["forked"]["cow_pairs"], "CoW pairs,",
          sp["forked"]["preemptions"], "preemptions")
    with open(os.path.join(HERE, "sampling_choices.json"), "w") as f:
        json.dump({"cases": sampling_cases()}, f)
    print("wrote fixtures; cfg0 steps", eng.total_steps,
          "min margin", min(min(v) for v in margins.values() if v))


if __name__ == "__main__":
    main()

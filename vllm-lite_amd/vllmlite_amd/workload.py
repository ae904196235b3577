"""Synthetic request mixes for the end-to-end benchmark.

`make_workload` draws the same requests as bench/bench.py:35-47 for a given
generator state: an optional shared prefix of uniform [32,126) ids, then per
request a lognormal prompt length (median 3*min_prompt, sigma 0.6) and output
length (median 3*min_out, sigma 0.7), both clipped and truncated to int, a BOS
(256) and uniform [32,126) body ids; greedy, ignore_eos. The draw order is the
reference's because the published token totals pin it.
"""

from __future__ import annotations

import numpy as np

from .request import SamplingParams

BOS = 256


def make_workload(n, rng, min_prompt, max_prompt, min_out, max_out, shared_prefix=0):
    prefix = [int(t) for t in rng.integers(32, 126, size=shared_prefix)] if shared_prefix else []
    reqs = []
    for i in range(n):
        plen = int(np.clip(rng.lognormal(np.log(min_prompt * 3), 0.6), min_prompt, max_prompt))
        olen = int(np.clip(rng.lognormal(np.log(min_out * 3), 0.7), min_out, max_out))
        body = [int(t) for t in rng.integers(32, 126, size=plen)]
        params = SamplingParams(max_tokens=olen, temperature=0.0, ignore_eos=True)
        reqs.append((f"r{i}", [BOS] + prefix + body, params))
    return reqs


def mixed_lengths(seed: int = 0, n: int = 48, shared_prefix: int = 0):
    """The 48-request ragged mix: prompts 16-256 (+BOS), outputs 16-192."""
    return make_workload(n, np.random.default_rng(seed), 16, 256, 16, 192, shared_prefix)


def shared_prefix_config(prefix_cache: bool = True):
    """The shared-prefix mix's engine as published (results/shared_prefix.json:2-17):
    TinyLlama 6 layers, d 384, H8/Hkv4, d_ff 1024, vocab 261, max_len 768;
    blocks of 16 with the same KV budget as 16 x 768 slots (768 blocks,
    bench/bench.py:156-157); 16 sequences, budget 1024."""
    from .config import CacheConfig, EngineConfig, ModelConfig, SchedulerConfig
    return EngineConfig(
        model=ModelConfig(n_layers=6, n_heads=8, n_kv_heads=4, d_model=384, d_ff=1024,
                          vocab_size=261, max_seq_len=768),
        cache=CacheConfig(block_size=16, num_blocks=768, enable_prefix_caching=prefix_cache),
        scheduler=SchedulerConfig(max_seqs=16, max_batched_tokens=1024))


def drive_forked(engine, reqs, suffix: str = ".c"):
    """The copy-on-write workload: submit `reqs`, and step the engine until it
    drains; after every step, each request that has just emitted its first
    token is forked once into `<id><suffix>`, a running copy sharing all of
    its blocks, partial tail included (BlockManager.fork,
    vllmlite/block_manager.py:133-137). Whichever of the two writes that tail
    first gets a copy-on-write pair (block_manager.py:74-85). Returns the
    forked request ids and those whose tail block was partial. The engine
    steps synchronously (the forks happen between steps)."""
    engine.lookahead = False
    for rid, ids, p in reqs:
        engine.add_request(params=p, request_id=rid, prompt_token_ids=ids)
    forked, partial = set(), []
    bs = engine.cfg.cache.block_size
    while engine.has_work:
        engine.step()
        for rid, filled in engine.just_started(suffix):
            if rid in forked:
                continue
            forked.add(rid)
            if filled % bs:
                partial.append(rid)
            engine.fork_request(rid, rid + suffix)
    return forked, partial

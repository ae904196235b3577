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

from .sequence import SamplingParams

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

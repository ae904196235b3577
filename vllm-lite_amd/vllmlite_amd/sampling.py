"""Choosing the next token from one row of logits.

The rules are the reference's (vllmlite/sampling.py:41-64), in this order:
EOS masked while fewer than min_tokens were generated; every token already
seen divided (if positive) or multiplied (if not) by the repetition penalty;
temperature 0 takes the argmax (ties to the lowest index); otherwise the
logits are divided by the temperature, cut to the top_k largest (top_k > 0),
cut to the smallest set of most probable tokens whose probability reaches
top_p (the token that crosses top_p kept; ranks from NumPy's default argsort
of the negated logits, so tied logits rank as the reference ranks them), and
one token is drawn from the renormalised distribution by the request's own
generator through `Generator.choice`, which consumes it as the reference's
draw does: the same seed gives the same tokens.
"""

from __future__ import annotations

import numpy as np


def _softmax(x: np.ndarray) -> np.ndarray:
    e = np.exp(x - x.max())
    return e / e.sum()


def choose(row: np.ndarray, params, seen, rng: np.random.Generator, num_generated: int,
           eos_id) -> int:
    x = np.array(row, dtype=np.float32)
    if eos_id is not None and num_generated < params.min_tokens:
        x[eos_id] = -np.inf
    pen = params.repetition_penalty
    if pen != 1.0 and len(seen):
        idx = np.unique(np.asarray(seen, dtype=np.int64))
        v = x[idx]
        x[idx] = np.where(v > 0, v / pen, v * pen)
    if params.temperature == 0.0:
        return int(np.argmax(x))
    x /= params.temperature
    k = params.top_k
    if 0 < k < x.size:
        x[x < np.partition(x, -k)[-k]] = -np.inf
    if params.top_p < 1.0:
        ranked = np.argsort(-x)
        w = _softmax(x[ranked])
        # mass ranked strictly ahead of each token; the one crossing top_p stays
        x[ranked[np.cumsum(w) - w >= params.top_p]] = -np.inf
    return int(rng.choice(x.size, p=_softmax(x)))

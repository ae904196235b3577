"""Greedy acceptance oracle (vllmlite/speculative.py:86-100) with the argmax
tie rule of numpy (lowest index; vllmlite/sampling.py:56-57). Test
infrastructure only."""

from __future__ import annotations

import numpy as np


def verify(logits: np.ndarray, drafts):
    """logits [len(drafts)+1, vocab] -> (tokens, accepted)."""
    picked = [int(np.argmax(logits[i])) for i in range(len(drafts) + 1)]
    out = []
    for i, d in enumerate(drafts):
        out.append(picked[i])
        if picked[i] != d:
            return out, i
    out.append(picked[len(drafts)])
    return out, len(drafts)

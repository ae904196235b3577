"""Speculative decoding with n-gram drafts and greedy acceptance.

NgramProposer: for the longest suffix of the context (prompt + outputs) of
length n in max_n..min_n that also occurs earlier, the tokens that followed
its last earlier occurrence are the drafts, up to k of them
(vllmlite/speculative.py:28-61). The search runs over the context packed as
little-endian int32 bytes with bytes.rfind, keeping only hits that start on a
token boundary.

Acceptance (vllmlite/speculative.py:86-100): with picked[i] the argmax of
row i, emit picked[i] while it equals draft i; at the first mismatch emit it
and stop (i drafts accepted); if every draft matched also emit picked[k].
"""

from __future__ import annotations

from typing import List, Sequence, Tuple

import numpy as np


class NgramProposer:
    def __init__(self, k: int = 4, min_n: int = 3, max_n: int = 8):
        self.k = k
        self.min_n = min_n
        self.max_n = max_n

    def propose(self, seq, k: int = None) -> List[int]:
        k = k or self.k
        toks = seq if isinstance(seq, list) else seq.context_ids()
        L = len(toks)
        hi = min(self.max_n, L - 1)
        if hi < self.min_n:
            return []
        packed = np.asarray(toks, dtype="<i4").tobytes()
        limit = 4 * (L - 1)  # an earlier occurrence ends before the last token
        for n in range(hi, self.min_n - 1, -1):
            needle = packed[4 * (L - n):]
            end = limit
            while True:
                at = packed.rfind(needle, 0, end)
                if at < 0:
                    break
                if at % 4 == 0:
                    i = at // 4 + n
                    return toks[i:i + k]
                end = at + len(needle) - 1
        return []


class SpecStats:
    def __init__(self):
        self.proposed = 0
        self.accepted = 0
        self.rounds = 0
        self.rounds_with_proposal = 0

    @property
    def acceptance_rate(self) -> float:
        return self.accepted / self.proposed if self.proposed else 0.0

    @property
    def tokens_per_round(self) -> float:
        return (self.accepted + self.rounds) / self.rounds if self.rounds else 0.0

    def as_dict(self) -> dict:
        return {"spec_proposed": self.proposed, "spec_accepted": self.accepted,
                "spec_acceptance_rate": round(self.acceptance_rate, 3),
                "spec_tokens_per_step": round(self.tokens_per_round, 3)}


def accept_greedy(picked: Sequence[int], drafts: Sequence[int]) -> Tuple[List[int], int]:
    """(tokens to emit, drafts accepted) from the rows' argmax ids."""
    k = len(drafts)
    p = [int(t) for t in picked[:k + 1]]
    for i in range(k):
        if p[i] != drafts[i]:
            return p[:i + 1], i
    return p, k


def verify(logits: np.ndarray, drafts: Sequence[int]) -> Tuple[List[int], int]:
    """accept_greedy on logits [k + 1, vocab]."""
    return accept_greedy(np.argmax(logits[:len(drafts) + 1], axis=-1), drafts)

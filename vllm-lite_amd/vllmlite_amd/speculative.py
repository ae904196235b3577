"""N-gram speculation and greedy acceptance.

`NgramProposer` and `SpecStats` follow vllmlite/speculative.py:28-83 (host-side
token search). `verify` is the greedy acceptance rule of speculative.py:86-100:
row i's argmax (ties to the lowest index) is emitted while it equals draft i;
the first mismatch is emitted and ends the run; if every draft matches, the
extra row's argmax is a free token. The GPU version of this rule is the
greedy-verify kernel (`ops.greedy_verify`).
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import numpy as np


class NgramProposer:
    def __init__(self, k: int = 4, min_n: int = 3, max_n: int = 8):
        self.k = k
        self.min_n = min_n
        self.max_n = max_n

    def propose(self, seq, k: Optional[int] = None) -> List[int]:
        k = k or self.k
        toks = seq.prompt_token_ids + seq.output_token_ids
        for n in range(min(self.max_n, len(toks) - 1), self.min_n - 1, -1):
            hit = self._rfind(toks, toks[-n:])
            if hit is None:
                continue
            guess = toks[hit + n:hit + n + k]
            if guess:
                return guess
        return []

    @staticmethod
    def _rfind(toks: List[int], pat: List[int]) -> Optional[int]:
        """Last occurrence of pat that is not the trailing one itself."""
        n = len(pat)
        for i in range(len(toks) - n - 1, -1, -1):
            if toks[i:i + n] == pat:
                return i
        return None


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
        return {
            "spec_proposed": self.proposed,
            "spec_accepted": self.accepted,
            "spec_acceptance_rate": round(self.acceptance_rate, 3),
            "spec_tokens_per_step": round(self.tokens_per_round, 3),
        }


def accept_greedy(picked, drafts) -> Tuple[List[int], int]:
    """The acceptance rule on precomputed per-row argmaxes."""
    out: List[int] = []
    for i, d in enumerate(drafts):
        out.append(int(picked[i]))
        if picked[i] != d:
            return out, i
    out.append(int(picked[len(drafts)]))
    return out, len(drafts)


def verify(logits: np.ndarray, drafts) -> Tuple[List[int], int]:
    """Returns (tokens_to_keep, num_drafts_accepted); always at least one token."""
    picked = np.argmax(logits[:len(drafts) + 1], axis=-1)
    return accept_greedy(picked, drafts)

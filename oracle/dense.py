"""Textbook dense causal attention with repeated KV heads, used to pin the
paged oracle (restates the checker of tests/test_attention.py:13-30).
Test infrastructure only."""

from __future__ import annotations

import numpy as np


def dense_attention(q, k, v, n_kv_heads: int, scale: float) -> np.ndarray:
    """q [q_len, H, D]; k, v [ctx, Hkv, D] in position order. Query i sits at
    ctx - q_len + i. Computed per head in float64 to be a stricter reference."""
    q_len, n_heads, _ = q.shape
    ctx = k.shape[0]
    rep = n_heads // n_kv_heads
    q64 = q.astype(np.float64)
    k64 = np.repeat(k.astype(np.float64), rep, axis=1)
    v64 = np.repeat(v.astype(np.float64), rep, axis=1)
    out = np.zeros(q.shape, dtype=np.float64)
    start = ctx - q_len
    for h in range(n_heads):
        s = (q64[:, h] @ k64[:, h].T) * scale
        for i in range(q_len):
            s[i, start + i + 1:] = -np.inf
        s = s - s.max(axis=-1, keepdims=True)
        e = np.exp(s)
        out[:, h] = (e / e.sum(axis=-1, keepdims=True)) @ v64[:, h]
    return out

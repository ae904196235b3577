"""Seeded ragged paged-attention batches shared by GPU tests and the bench.

A batch is a list of (q_len, ctx) per sequence. Block tables are consecutive
slices of a seeded permutation of the block pool, so blocks are scattered and
out of order. Every cache slot a sequence does not own is NaN (bf16/fp32), so
a kernel that reads outside the table or past ctx produces NaN and fails.
"""

from __future__ import annotations

import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 to the nearest bf16 (ties to even), returned as fp32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def make_batch(seqs, H, Hkv, D, block_size, num_blocks=None, seed=0, poison=True):
    rng = np.random.default_rng(seed)
    bs = block_size
    nbs = [-(-ctx // bs) for _, ctx in seqs]
    if num_blocks is None:
        num_blocks = sum(nbs) + 7
    perm = rng.permutation(num_blocks)
    tables, off = [], 0
    for nb in nbs:
        tables.append(perm[off:off + nb].astype(np.int32))
        off += nb
    W = max(1, max(nbs))
    bt = np.zeros((len(seqs), W), np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    slots = num_blocks * bs
    ck = np.full((slots, Hkv, D), np.nan, np.float32) if poison else np.zeros((slots, Hkv, D), np.float32)
    cv = ck.copy()
    for (q, ctx), t in zip(seqs, tables):
        s = (t[:, None].astype(np.int64) * bs + np.arange(bs)[None, :]).reshape(-1)[:ctx]
        ck[s] = rng.standard_normal((ctx, Hkv, D)).astype(np.float32)
        cv[s] = rng.standard_normal((ctx, Hkv, D)).astype(np.float32)
    T = sum(q for q, _ in seqs)
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    qsl = np.zeros(len(seqs) + 1, np.int32)
    qsl[1:] = np.cumsum([q_ for q_, _ in seqs])
    seq_lens = np.array([c for _, c in seqs], np.int32)
    return dict(q=q, k_cache=ck, v_cache=cv, block_tables=bt, seq_lens=seq_lens, qsl=qsl,
                tables=tables, H=H, Hkv=Hkv, D=D, bs=bs, scale=1.0 / np.sqrt(D))


def oracle_attention(b, q=None, ck=None, cv=None):
    """Per-sequence oracle paged_attention over the batch (fp32)."""
    from oracle.attention import gather_slots, paged_attention
    q = b["q"] if q is None else q
    ck = b["k_cache"] if ck is None else ck
    cv = b["v_cache"] if cv is None else cv
    out = np.zeros_like(q)
    for i, t in enumerate(b["tables"]):
        s0, s1 = b["qsl"][i], b["qsl"][i + 1]
        if s1 == s0:
            continue
        slots = gather_slots(t, b["bs"], int(b["seq_lens"][i]))
        out[s0:s1] = paged_attention(q[s0:s1], ck, cv, slots, b["Hkv"], b["scale"])
    return out


def head_major(cache: np.ndarray, bs: int) -> np.ndarray:
    """A token-major cache [slots, Hkv, D] rearranged as head-major blocks
    [blocks, Hkv, bs, D]: the same values, only the order of the rows inside
    each block differs (slot = block * bs + offset in both)."""
    s, hkv, d = cache.shape
    return np.ascontiguousarray(cache.reshape(s // bs, bs, hkv, d).transpose(0, 2, 1, 3))


def token_major(cache: np.ndarray) -> np.ndarray:
    """The inverse of head_major: [blocks, Hkv, bs, D] -> [slots, Hkv, D]."""
    nb, hkv, bs, d = cache.shape
    return np.ascontiguousarray(cache.transpose(0, 2, 1, 3).reshape(nb * bs, hkv, d))

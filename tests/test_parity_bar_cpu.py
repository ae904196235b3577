"""The bf16 row bar can fail: an output that lost part of its context is
rejected, while bf16 rounding noise of the right size is accepted.

The cases are the long contexts of the workloads: one spec-verify sequence
with 32768 cached keys (5 queries, 32 query heads over 8 KV heads, head_dim
128) and one decode sequence with 8192 keys, with bf16-valued N(0,1) Q/K/V.
Keys are dropped either at random (1/16 of them) or as one contiguous 1/16 of
the context, which is what a lost split partition looks like. The oracle's
output computed without them must fail the bar on every trial.
"""

import numpy as np
import pytest

from batches import bf16_round
from oracle.attention import paged_attention
from parity import BF16_ROW_REL, assert_rows_close, row_rel_err

H, HKV, D = 32, 8, 128


def _case(ctx, q_len, seed):
    rng = np.random.default_rng(seed)
    k = bf16_round(rng.standard_normal((ctx, HKV, D)).astype(np.float32))
    v = bf16_round(rng.standard_normal((ctx, HKV, D)).astype(np.float32))
    q = bf16_round(rng.standard_normal((q_len, H, D)).astype(np.float32))
    return rng, q, k, v


def _attend(q, k, v, keep):
    return paged_attention(q, k, v, keep, HKV, 1.0 / np.sqrt(D))


@pytest.mark.parametrize("ctx,q_len", [(32768, 5), (8192, 1)])
@pytest.mark.parametrize("trial", range(2))
def test_bar_rejects_lost_keys(ctx, q_len, trial):
    rng, q, k, v = _case(ctx, q_len, trial)
    want = _attend(q, k, v, np.arange(ctx))
    # keys before the first query position only, so every query keeps its causal tail
    lo = ctx - q_len
    drop_random = np.sort(rng.choice(lo, size=ctx // 16, replace=False))
    start = int(rng.integers(0, lo - ctx // 16))
    drop_range = np.arange(start, start + ctx // 16)
    for drop in (drop_random, drop_range):
        keep = np.setdiff1d(np.arange(ctx), drop)
        lost = _attend(q, k, v, keep)
        assert row_rel_err(lost, want).max() > BF16_ROW_REL
        with pytest.raises(AssertionError):
            assert_rows_close(lost, want, BF16_ROW_REL)


@pytest.mark.parametrize("ctx,q_len", [(32768, 5), (8192, 1)])
def test_bar_accepts_bf16_rounding(ctx, q_len):
    """The kernels' own error sources at their size: probabilities rounded to
    bf16 before the PV product, and the bf16 store of the output."""
    _, q, k, v = _case(ctx, q_len, 7)
    want = _attend(q, k, v, np.arange(ctx))
    scale = 1.0 / np.sqrt(D)
    rep = H // HKV
    qg = q.transpose(1, 0, 2).reshape(HKV, rep * q_len, D)
    s = np.matmul(qg, k.transpose(1, 2, 0)) * scale
    if q_len > 1:
        qpos = np.arange(ctx - q_len, ctx)[:, None]
        s = s.reshape(HKV, rep, q_len, ctx)
        s[:, :, np.arange(ctx)[None, :] > qpos] = -np.inf
        s = s.reshape(HKV, rep * q_len, ctx)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    l = p.sum(axis=-1, keepdims=True)
    noisy = np.matmul(bf16_round(p), v.transpose(1, 0, 2)) / l
    noisy = bf16_round(noisy.reshape(H, q_len, D).transpose(1, 0, 2))
    assert_rows_close(noisy, want, BF16_ROW_REL)

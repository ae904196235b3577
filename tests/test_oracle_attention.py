"""Pins the oracle's attention, slot and RoPE functions (oracle/attention.py).

The grid and tolerance are the reference's own (tests/test_attention.py:33-57);
the known answers are tests/test_attention.py:60-77. Closed forms added here
catch what a grid of random inputs might not: one visible key, identical keys,
and a RoPE rotation built independently with math.cos/math.sin.
"""

import math

import numpy as np
import pytest

from oracle.attention import apply_rope, build_rope, gather_slots, paged_attention, write_kv
from oracle.dense import dense_attention


@pytest.mark.parametrize("q_len", [1, 5, 17])
@pytest.mark.parametrize("n_heads,n_kv_heads", [(4, 4), (8, 2), (6, 1)])
@pytest.mark.parametrize("block_size", [1, 4, 16])
def test_paged_matches_dense(q_len, n_heads, n_kv_heads, block_size):
    rng = np.random.default_rng(0)
    d, ctx = 8, 37
    nb = (ctx + block_size - 1) // block_size
    total = nb + 5
    ck = rng.standard_normal((total * block_size, n_kv_heads, d)).astype(np.float32)
    cv = rng.standard_normal((total * block_size, n_kv_heads, d)).astype(np.float32)
    table = list(rng.permutation(total)[:nb])
    slots = gather_slots(table, block_size, ctx)
    q = rng.standard_normal((q_len, n_heads, d)).astype(np.float32)
    scale = 1.0 / np.sqrt(d)
    got = paged_attention(q, ck, cv, slots, n_kv_heads, scale)
    want = dense_attention(q, ck[slots], cv[slots], n_kv_heads, scale)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


def test_gather_slots_follows_the_table():
    assert list(gather_slots([3, 0], block_size=4, count=6)) == [12, 13, 14, 15, 0, 1]


def test_gather_slots_brute_force():
    rng = np.random.default_rng(1)
    for bs in (1, 3, 16):
        table = list(rng.permutation(40)[:7])
        for count in (0, 1, bs, 7 * bs - 1, 7 * bs):
            want = [table[p // bs] * bs + p % bs for p in range(count)]
            assert list(gather_slots(table, bs, count)) == want


def test_write_kv_scatters_rows():
    ck = np.zeros((10, 2, 3), np.float32)
    cv = np.zeros((10, 2, 3), np.float32)
    k = np.arange(12, dtype=np.float32).reshape(2, 2, 3)
    write_kv(ck, cv, k, -k, np.array([7, 2]))
    assert (ck[7] == k[0]).all() and (ck[2] == k[1]).all() and (cv[2] == -k[1]).all()
    assert ck[[0, 1, 3, 4, 5, 6, 8, 9]].sum() == 0


def test_single_key_returns_its_value():
    rng = np.random.default_rng(2)
    ck = rng.standard_normal((4, 2, 8)).astype(np.float32)
    cv = rng.standard_normal((4, 2, 8)).astype(np.float32)
    q = rng.standard_normal((1, 4, 8)).astype(np.float32)
    out = paged_attention(q, ck, cv, np.array([3]), 2, 0.5)
    # head h reads kv head h // 2
    np.testing.assert_allclose(out[0], cv[3][[0, 0, 1, 1]], rtol=1e-6)


def test_identical_keys_average_the_values():
    rng = np.random.default_rng(3)
    ck = np.repeat(rng.standard_normal((1, 1, 8)).astype(np.float32), 6, axis=0)
    cv = rng.standard_normal((6, 1, 8)).astype(np.float32)
    q = rng.standard_normal((1, 2, 8)).astype(np.float32)
    out = paged_attention(q, ck, cv, np.arange(6), 1, 0.3)
    np.testing.assert_allclose(out[0, 0], cv[:, 0].mean(0), rtol=1e-5)


def test_causal_first_query_sees_only_the_prefix():
    rng = np.random.default_rng(4)
    ck = rng.standard_normal((9, 1, 4)).astype(np.float32)
    cv = rng.standard_normal((9, 1, 4)).astype(np.float32)
    q = rng.standard_normal((3, 1, 4)).astype(np.float32)
    full = paged_attention(q, ck, cv, np.arange(9), 1, 0.5)
    # query 0 sits at position 6 and must equal decode over slots 0..6
    dec = paged_attention(q[:1], ck, cv, np.arange(7), 1, 0.5)
    np.testing.assert_allclose(full[0], dec[0], rtol=1e-6)


def test_rope_is_position_dependent():
    cos, sin = build_rope(8, 16)
    x = np.ones((2, 1, 8), dtype=np.float32)
    a = apply_rope(x, np.array([0, 0]), cos, sin)
    b = apply_rope(x, np.array([0, 5]), cos, sin)
    np.testing.assert_allclose(a[0], b[0])
    assert not np.allclose(a[1], b[1])


def test_position_zero_is_identity():
    cos, sin = build_rope(8, 16)
    x = np.random.default_rng(0).standard_normal((1, 2, 8)).astype(np.float32)
    np.testing.assert_allclose(apply_rope(x, np.array([0]), cos, sin), x, atol=1e-6)


def test_rope_is_an_interleaved_rotation():
    """Pairs (2i, 2i+1) rotate by pos * 10000^(-2i/D); not the half-split form."""
    d, pos = 8, 11
    cos, sin = build_rope(d, 32)
    x = np.random.default_rng(5).standard_normal((1, 1, d)).astype(np.float32)
    got = apply_rope(x, np.array([pos]), cos, sin)[0, 0]
    for i in range(d // 2):
        a = pos * 10000.0 ** (-(2 * i) / d)
        e, o = float(x[0, 0, 2 * i]), float(x[0, 0, 2 * i + 1])
        assert abs(got[2 * i] - (e * math.cos(a) - o * math.sin(a))) < 1e-5
        assert abs(got[2 * i + 1] - (e * math.sin(a) + o * math.cos(a))) < 1e-5
    np.testing.assert_allclose(np.linalg.norm(got), np.linalg.norm(x), rtol=1e-5)

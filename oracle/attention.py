"""NumPy restatement of vllmlite/attention.py:21-98. Test infrastructure only.

The operations, their shapes and their order are the reference's, so that the
fp32 results (and the CPU time) are those of the reference.
"""

from __future__ import annotations

import numpy as np


def build_rope(head_dim: int, max_pos: int, theta: float = 10000.0):
    """attention.py:21-25: fp32 angle table pos * theta^(-2i/D); returns (cos, sin) [max_pos, D/2]."""
    inv = 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float32) / head_dim))
    ang = np.arange(max_pos, dtype=np.float32)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def apply_rope(x: np.ndarray, positions: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """attention.py:28-37: rotate interleaved (even, odd) pairs of each head. x [T, H, D]."""
    c = cos[positions][:, None, :]
    s = sin[positions][:, None, :]
    even = x[..., 0::2]
    odd = x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = even * c - odd * s
    out[..., 1::2] = even * s + odd * c
    return out


def gather_slots(block_ids, block_size: int, count: int) -> np.ndarray:
    """attention.py:40-44: flat slots of positions 0..count-1 through a block table."""
    bids = np.asarray(block_ids, dtype=np.int64)
    return (bids[:, None] * block_size + np.arange(block_size, dtype=np.int64)[None, :]).reshape(-1)[:count]


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> the nearest bfloat16 (ties to even), returned as fp32: the
    values a bf16 K/V cache holds. No reference counterpart (the reference
    caches fp32, attention.py:47-49); pinned in tests/test_oracle_bf16.py by
    torch's bfloat16 conversion and hand-picked ties. NaN stays NaN."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a), a, r).astype(np.float32)


def fp8_e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """OCP FP8 E4M3 ("e4m3fn") bytes -> fp32, from the format's definition:
    sign bit, 4 exponent bits with bias 7, 3 mantissa bits; exponent 0 is
    subnormal (m * 2^-9); 0x7F / 0xFF are NaN; there are no infinities. No
    reference counterpart (the reference caches fp32); pinned in
    tests/test_oracle_fp8.py."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    e, m = (c >> 3) & 15, c & 7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e - 7))
    mag = np.where((c & 0x7F) == 0x7F, np.nan, mag)
    return np.where(c & 0x80, -mag, mag).astype(np.float32)


_FP8_VALUES = fp8_e4m3_decode(np.arange(0x7F, dtype=np.uint8))  # 0, 2^-9, ..., 448


def fp8_e4m3_encode(x: np.ndarray) -> np.ndarray:
    """fp32 -> OCP FP8 E4M3 bytes, round to nearest with ties to the even
    code (the one whose mantissa's last bit is 0), saturating: finite values
    and infinities beyond 448 in magnitude become +-448; NaN becomes 0x7F
    (0xFF if negative). Found by a search over the 127 non-negative finite
    values, not by bit manipulation, so it is independent of the kernels'
    method."""
    a = np.asarray(x, dtype=np.float32)
    mag = np.minimum(np.abs(a).astype(np.float64), 448.0)
    hi = np.searchsorted(_FP8_VALUES, mag, side="left").clip(0, 126)   # first value >= mag
    lo = np.maximum(hi - 1, 0)
    d_lo, d_hi = mag - _FP8_VALUES[lo], _FP8_VALUES[hi] - mag
    pick = np.where(d_lo < d_hi, lo, np.where(d_hi < d_lo, hi, np.where(lo % 2 == 0, lo, hi)))
    pick = np.where(_FP8_VALUES[hi] == mag, hi, pick)
    code = pick.astype(np.uint8) | np.where(np.signbit(a), 0x80, 0).astype(np.uint8)
    return np.where(np.isnan(a), np.where(np.signbit(a), 0xFF, 0x7F), code).astype(np.uint8)


def round_fp8_e4m3(x: np.ndarray) -> np.ndarray:
    """The values an FP8 E4M3 K/V cache holds: fp8_e4m3_encode then decode."""
    return fp8_e4m3_decode(fp8_e4m3_encode(x))


def write_kv(cache_k, cache_v, k, v, slots) -> None:
    """attention.py:47-49: scatter rows into the flat [slots, Hkv, D] cache."""
    cache_k[slots] = k
    cache_v[slots] = v


def softmax_(x: np.ndarray) -> np.ndarray:
    """attention.py:52-56, in place over the last axis."""
    x -= x.max(axis=-1, keepdims=True)
    np.exp(x, out=x)
    x /= x.sum(axis=-1, keepdims=True)
    return x


def paged_attention(q, cache_k, cache_v, read_slots, n_kv_heads: int, scale: float) -> np.ndarray:
    """attention.py:59-98, one sequence. q [q_len, H, D]; read_slots are all
    ctx slots of the sequence in position order; query j sits at position
    ctx - q_len + j and sees keys 0..that position (mask only when q_len > 1)."""
    q_len, n_heads, d = q.shape
    ctx = read_slots.shape[0]
    rep = n_heads // n_kv_heads
    k = cache_k[read_slots]
    v = cache_v[read_slots]
    qg = q.transpose(1, 0, 2).reshape(n_kv_heads, rep * q_len, d)
    scores = np.matmul(qg, k.transpose(1, 2, 0))
    scores *= scale
    if q_len > 1:
        qpos = np.arange(ctx - q_len, ctx)[:, None]
        kpos = np.arange(ctx)[None, :]
        scores = scores.reshape(n_kv_heads, rep, q_len, ctx)
        scores[:, :, kpos > qpos] = -np.inf
        scores = scores.reshape(n_kv_heads, rep * q_len, ctx)
    softmax_(scores)
    out = np.matmul(scores, v.transpose(1, 0, 2))
    return out.reshape(n_heads, q_len, d).transpose(1, 0, 2)

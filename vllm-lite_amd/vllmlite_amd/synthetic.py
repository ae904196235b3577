"""Seeded synthetic batches for the paged-attention step, built on the device.

A batch is a list of (query tokens, context) per sequence: sequence i attends
keys 0..ctx_i-1 and its q_i query tokens sit at positions ctx_i-q_i..ctx_i-1
(vllmlite/attention.py:69-71). Block tables are consecutive slices of a seeded
permutation of a large block pool, so blocks are scattered and out of order;
every slot a sequence does not own is NaN, as are the slots of this step's new
tokens until reshape_and_cache writes them, so a stray read or a missing write
shows up as NaN.

The workloads:
  decode_256     256 sequences x 1 query, context lognormal (median 1024,
                 sigma 0.6) clipped to 64..8192
  mixed_8392     16 prefill chunks of 512 tokens with 0..2048 prior context
                 (uniform) after 200 decodes with context 128..4096 (uniform);
                 decodes first, as the scheduler orders running sequences
  verify_64x5    64 sequences x 5 query positions (4 drafts + 1), context
                 uniform 1024..32768
all with 32 query heads over 8 KV heads, head_dim 128, bf16, block size 16,
in a 2^17-block pool (4 GiB per K and V, far above the 256 MB Infinity Cache).
"""

from __future__ import annotations

import numpy as np

H, HKV, D, BS, POOL = 32, 8, 128, 16, 1 << 17


def decode_256_seqs(seed=0, n=256, sigma=0.6):
    rng = np.random.default_rng(seed)
    ctx = np.clip(np.rint(rng.lognormal(np.log(1024.0), sigma, size=n)), 64, 8192).astype(np.int64)
    return [(1, int(c)) for c in ctx]


def mixed_8392_seqs(seed=0):
    rng = np.random.default_rng(seed)
    prior = rng.integers(0, 2049, size=16)
    dec = rng.integers(128, 4097, size=200)
    return [(1, int(c)) for c in dec] + [(512, int(p) + 512) for p in prior]


def verify_64x5_seqs(seed=0):
    rng = np.random.default_rng(seed)
    ctx = rng.integers(1024, 32769, size=64)
    return [(5, int(c)) for c in ctx]


def build(torch, seqs, seed=0, pool_blocks=POOL, dtype=None, heads=(H, HKV, D), bs=BS,
          device="cuda"):
    """Device tensors of a batch. Prior context (positions < ctx - q) is
    filled with N(0,1) values; the q new tokens' K/V are returned separately
    (knew, vnew) with their slot_mapping for reshape_and_cache."""
    dtype = dtype or torch.bfloat16
    nh, nkv, hd = heads
    rng = np.random.default_rng(seed + 1)
    q_lens = np.array([q for q, _ in seqs], np.int64)
    ctx = np.array([c for _, c in seqs], np.int64)
    nblk = (ctx + bs - 1) // bs
    if int(nblk.sum()) > pool_blocks:
        raise ValueError("pool too small for the batch")
    perm = rng.permutation(pool_blocks).astype(np.int64)
    S = len(seqs)
    W = int(nblk.max())
    tables = np.zeros((S, W), np.int32)
    off = 0
    prior_slots, new_slots = [], []
    for i in range(S):
        t = perm[off:off + nblk[i]]
        off += nblk[i]
        tables[i, :nblk[i]] = t
        slots = (t[:, None] * bs + np.arange(bs)[None, :]).reshape(-1)[:ctx[i]]
        prior_slots.append(slots[:ctx[i] - q_lens[i]])
        new_slots.append(slots[ctx[i] - q_lens[i]:])
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    kc = torch.full((pool_blocks * bs, nkv, hd), float("nan"), dtype=dtype, device=device)
    vc = torch.full_like(kc, float("nan"))
    ps = torch.from_numpy(np.concatenate(prior_slots)).to(device)
    n = ps.numel()
    if n:
        kc[ps] = torch.randn((n, nkv, hd), generator=g, device=device).to(dtype)
        vc[ps] = torch.randn((n, nkv, hd), generator=g, device=device).to(dtype)
    T = int(q_lens.sum())
    q = torch.randn((T, nh, hd), generator=g, device=device).to(dtype)
    knew = torch.randn((T, nkv, hd), generator=g, device=device).to(dtype)
    vnew = torch.randn((T, nkv, hd), generator=g, device=device).to(dtype)
    qsl = np.zeros(S + 1, np.int32)
    qsl[1:] = np.cumsum(q_lens)
    return dict(
        seqs=seqs, q_lens=q_lens, ctx=ctx, tables_np=tables, H=nh, Hkv=nkv, D=hd, bs=bs,
        q=q, kc=kc, vc=vc, knew=knew, vnew=vnew,
        slot_mapping=torch.from_numpy(np.concatenate(new_slots).astype(np.int32)).to(device),
        bt=torch.from_numpy(tables).to(device),
        seq_lens=torch.from_numpy(ctx.astype(np.int32)).to(device),
        qsl=torch.from_numpy(qsl).to(device), qsl_np=qsl, scale=1.0 / np.sqrt(hd),
        max_q=int(q_lens.max()), min_q=int(q_lens[q_lens > 0].min()) if (q_lens > 0).any() else 0)


def to_head_major(cache, bs):
    """A token-major cache [slots, Hkv, D] as a new head-major tensor
    [blocks, Hkv, bs, D] (the same rows; slot = block * bs + offset)."""
    s, hkv, d = cache.shape
    return cache.view(s // bs, bs, hkv, d).permute(0, 2, 1, 3).contiguous()


def to_token_major(cache):
    """The inverse of to_head_major: [blocks, Hkv, bs, D] -> [slots, Hkv, D]."""
    nb, hkv, bs, d = cache.shape
    return cache.permute(0, 2, 1, 3).reshape(nb * bs, hkv, d).contiguous()


def algorithmic_bytes(b, with_scatter=True):
    """Each K/V element once, Q read and out written once, block-table
    entries and lengths; plus, with the scatter, the new K/V read and
    written once and the slot mapping read."""
    es = 2 if b["q"].dtype.itemsize == 2 else 4
    ctx, T = b["ctx"], int(b["q_lens"].sum())
    H_, Hkv_, D_ = b["H"], b["Hkv"], b["D"]
    attn = (int(ctx.sum()) * 2 * Hkv_ * D_ * es + 2 * T * H_ * D_ * es
            + int(((ctx + b["bs"] - 1) // b["bs"]).sum()) * 4 + 4 * len(ctx) + 4 * (len(ctx) + 1))
    scatter = 2 * (2 * T * Hkv_ * D_ * es) + 4 * T
    return attn + (scatter if with_scatter else 0)


def attention_flops(b):
    """4 * head_dim flops per unmasked (query, key) pair and query head
    (QK^T and PV)."""
    q, c = b["q_lens"], b["ctx"]
    pairs = q * (c - q) + q * (q + 1) // 2
    return int(pairs.sum()) * b["H"] * b["D"] * 4


def torch_reference_check(torch, b, out, idx):
    """Sequences `idx` of the batch against a plain fp32 PyTorch attention
    over the same gathered K/V (a sanity check for benchmarks; parity with
    the reference is established by the tests). Returns the worst max-abs
    error relative to the reference's largest magnitude (inf on NaN)."""
    worst = 0.0
    qsl = b["qsl_np"]
    rep = b["H"] // b["Hkv"]
    for i in idx:
        c, ql = int(b["ctx"][i]), int(b["q_lens"][i])
        nb = (c + b["bs"] - 1) // b["bs"]
        blocks = torch.from_numpy(b["tables_np"][i, :nb].astype(np.int64)).to(b["kc"].device)
        slots = (blocks[:, None] * b["bs"] + torch.arange(b["bs"], device=blocks.device)).reshape(-1)[:c]
        k = b["kc"][slots].float().repeat_interleave(rep, dim=1)  # [c, H, D]
        v = b["vc"][slots].float().repeat_interleave(rep, dim=1)
        qq = b["q"][qsl[i]:qsl[i + 1]].float()                     # [ql, H, D]
        s_ = torch.einsum("qhd,khd->hqk", qq, k) * b["scale"]
        pos = torch.arange(c - ql, c, device=k.device)[:, None]
        s_ = s_.masked_fill(torch.arange(c, device=k.device)[None, :] > pos, float("-inf"))
        want = torch.einsum("hqk,khd->qhd", torch.softmax(s_, dim=-1), v)
        got = out[qsl[i]:qsl[i + 1]].float()
        if not torch.isfinite(got).all():
            return float("inf")
        worst = max(worst, float((got - want).abs().max() / want.abs().max().clamp_min(1e-6)))
    return worst

"""GPU parity of every kernel against the oracle, through the C ABI.

Bars: copies and scatters bit-exact; fp32 attention rtol 1e-4 / atol 1e-5
(the reference's own tolerance, tests/test_attention.py:57) and every (token,
head) row within 1e-4 normwise; bf16 attention every row within 2e-2 normwise
against fp32 oracle math on bf16-rounded inputs (tests/parity.py); argmax and
greedy acceptance exact.
"""

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from batches import bf16_round, head_major, make_batch, oracle_attention, token_major  # noqa: E402
from parity import BF16_ROW_REL, F32_ROW_REL, assert_rows_close  # noqa: E402

pytestmark = pytest.mark.gpu


def ops():
    from vllmlite_amd import ops as o
    return o


def dev(x, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    return t if dtype is None else t.to(dtype)


def to_np(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def caches(b, tdt, layout="token"):
    """The batch's K/V caches on the device, token-major [slots, Hkv, D] or
    head-major [blocks, Hkv, bs, D]."""
    if layout == "head":
        return tuple(dev(head_major(b[n], b["bs"]), tdt) for n in ("k_cache", "v_cache"))
    return dev(b["k_cache"], tdt), dev(b["v_cache"], tdt)


def run_attention(b, dtype, ws_bytes=None, exact_max_q=True, exact_min_q=True, ctx_hint=False,
                  layout="token"):
    """exact_max_q / exact_min_q / ctx_hint: pass the batch's true query-count
    and context bounds (they choose the launches) or 0 (the kernels decide on
    the device); layout: the caches token-major or head-major."""
    o = ops()
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    q = dev(b["q"], tdt)
    kc, vc = caches(b, tdt, layout)
    out = torch.empty_like(q)
    S, T = len(b["seq_lens"]), b["q"].shape[0]
    if ws_bytes is None:
        ws_bytes = o.paged_attention_workspace_size(S, T, b["H"], b["D"], int(b["seq_lens"].max()))
    ws = o.AttentionWorkspace().get(ws_bytes)
    q_lens = np.diff(b["qsl"])
    max_q, min_q = int(q_lens.max()), int(q_lens[q_lens > 0].min())
    o.paged_attention(out, q, kc, vc, dev(b["block_tables"]), dev(b["seq_lens"]), dev(b["qsl"]),
                      b["scale"], b["bs"], ws, max_query_len=max_q if exact_max_q else 0,
                      min_query_len=min_q if exact_min_q else 0,
                      max_context_len=int(b["seq_lens"].max()) if ctx_hint else 0)
    return to_np(out)


def expected(b, dtype):
    if dtype == "f32":
        return oracle_attention(b)
    return oracle_attention(b, bf16_round(b["q"]), bf16_round(b["k_cache"]), bf16_round(b["v_cache"]))


def check(got, want, dtype):
    assert np.isfinite(got).all()
    if dtype == "f32":
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)
        assert_rows_close(got, want, F32_ROW_REL)
    else:
        assert_rows_close(got, want, BF16_ROW_REL)


# -- the reference's grid (tests/test_attention.py:33-57), one sequence per launch
@pytest.mark.parametrize("q_len", [1, 5, 17])
@pytest.mark.parametrize("H,Hkv", [(4, 4), (8, 2), (6, 1)])
@pytest.mark.parametrize("bs", [1, 4, 16])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_reference_grid(q_len, H, Hkv, bs, dtype):
    b = make_batch([(q_len, 37)], H, Hkv, 8, bs, seed=0)
    check(run_attention(b, dtype), expected(b, dtype), dtype)


MIXED = [(1, 1), (1, 37), (5, 40), (17, 17), (1, 300), (64, 700), (3, 1025), (1, 16), (9, 33)]


@pytest.mark.parametrize("layout", ["token", "head"])
@pytest.mark.parametrize("hints", ["both", "max", "none"])
@pytest.mark.parametrize("shape", [(8, 4, 48), (32, 8, 128), (4, 2, 16), (6, 3, 64)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_mixed_prefill_decode_one_launch(shape, dtype, hints, layout):
    """Decodes and multi-query sequences in one call. With both bounds known
    the bf16 fast shapes launch the step kernel alone; with only the maximum,
    the step kernel and the tile kernels (each takes its items from the
    plan); with neither, the step kernel takes every item. Both cache
    layouts."""
    H, Hkv, D = shape
    b = make_batch(MIXED, H, Hkv, D, 16, seed=1)
    got = run_attention(b, dtype, exact_max_q=hints != "none", exact_min_q=hints == "both",
                        layout=layout)
    check(got, expected(b, dtype), dtype)


def test_query_bounds_are_checked():
    o = ops()
    b = make_batch([(3, 40)], 4, 4, 64, 16, seed=4)
    with pytest.raises(RuntimeError, match="query length bounds"):
        q = dev(b["q"], torch.bfloat16)
        kc = dev(b["k_cache"], torch.bfloat16)
        ws = o.AttentionWorkspace().get(o.paged_attention_workspace_size(1, 3, 4, 64, 40))
        o.paged_attention(torch.empty_like(q), q, kc, kc, dev(b["block_tables"]),
                          dev(b["seq_lens"]), dev(b["qsl"]), b["scale"], 16, ws,
                          max_query_len=3, min_query_len=4)


@pytest.mark.parametrize("layout", ["token", "head"])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_long_context_split_and_small_workspace(dtype, layout):
    b = make_batch([(1, 5000), (4, 3000), (1, 70)], 8, 2, 64, 16, seed=2)
    want = expected(b, dtype)
    check(run_attention(b, dtype, layout=layout), want, dtype)
    # a workspace with room for the plan only: no context splitting at all
    o = ops()
    check(run_attention(b, dtype, ws_bytes=o.lib().vl_paged_attention_min_workspace(3),
                        layout=layout), want, dtype)


def test_bad_arguments_raise():
    o = ops()
    b = make_batch([(1, 20)], 6, 3, 8, 4)
    q = dev(b["q"])
    kc = dev(b["k_cache"])
    out = torch.empty_like(q)
    ws = o.AttentionWorkspace().get(1 << 16)
    with pytest.raises(ValueError):
        o.paged_attention(out, q, kc, kc, dev(b["block_tables"]), dev(b["seq_lens"]),
                          dev(b["qsl"][:1]), b["scale"], b["bs"], ws)
    rc = o.lib().vl_paged_attention(None, None, 0, None, None, None, 0, None, None, 1, 1, 6, 4, 8,
                                    4, 1.0, 0, 0, 0, 0, 0, None, 0, None)
    assert rc == -1 and b"multiple" in o.lib().vl_last_error()


@pytest.mark.parametrize("layout", ["token", "head"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float8_e4m3fn])
def test_reshape_and_cache_bit_exact(dtype, layout):
    """The scatter equals oracle.write_kv bit for bit; a head-major cache
    holds the same rows (head_major of the oracle's token-major cache)."""
    from oracle.attention import write_kv
    o = ops()
    rng = np.random.default_rng(3)
    T, Hkv, D, slots = 77, 4, 48, 512
    qkv = torch.from_numpy(rng.standard_normal((T, (8 + 2 * Hkv) * D)).astype(np.float32)).to(dtype)
    k = qkv[:, 8 * D:(8 + Hkv) * D].view(T, Hkv, D)
    v = qkv[:, (8 + Hkv) * D:].view(T, Hkv, D)
    slot = rng.permutation(slots)[:T].astype(np.int32)
    kc = torch.from_numpy(rng.standard_normal((slots, Hkv, D)).astype(np.float32)).to(dtype)
    vc = (kc.float() * 2).to(dtype)
    want_k, want_v = kc.clone().float().numpy(), vc.clone().float().numpy()
    write_kv(want_k, want_v, k.float().numpy(), v.float().numpy(), slot)
    dqkv = qkv.cuda()
    dk = dqkv[:, 8 * D:(8 + Hkv) * D].view(T, Hkv, D)
    dv = dqkv[:, (8 + Hkv) * D:].view(T, Hkv, D)
    if layout == "head":
        dkc, dvc = (dev(head_major(x.float().numpy(), 16), dtype) for x in (kc, vc))
        want_k, want_v = head_major(want_k, 16), head_major(want_v, 16)
    else:
        dkc, dvc = kc.cuda(), vc.cuda()
    o.reshape_and_cache(dk, dv, dkc, dvc, dev(slot))
    assert np.array_equal(to_np(dkc), want_k) and np.array_equal(to_np(dvc), want_v)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float8_e4m3fn])
def test_copy_blocks_bit_exact(dtype):
    from oracle.runner import NumpyRunner
    from vllmlite_amd.config import CacheConfig, ModelConfig
    o = ops()
    mc = ModelConfig(n_layers=3, n_heads=8, n_kv_heads=4, d_model=384, d_ff=64, max_seq_len=64)
    cc = CacheConfig(block_size=16, num_blocks=100)
    r = NumpyRunner(mc, cc)
    rng = np.random.default_rng(4)
    r.cache_k[...] = rng.standard_normal(r.cache_k.shape)
    r.cache_v[...] = rng.standard_normal(r.cache_v.shape)
    r.cache_k[...] = torch.from_numpy(r.cache_k).to(dtype).float().numpy()
    r.cache_v[...] = torch.from_numpy(r.cache_v).to(dtype).float().numpy()
    dk, dv = dev(r.cache_k, dtype), dev(r.cache_v, dtype)
    # 48 pairs, several sharing a source, destinations distinct and never a source
    srcs = rng.integers(0, 20, size=48)
    dsts = 20 + rng.permutation(80)[:48]
    pairs = [(int(s), int(d)) for s, d in zip(srcs, dsts)]
    # the same copies on head-major caches [L, blocks, Hkv, 16, D]
    hk = torch.stack([dev(head_major(x, 16), dtype) for x in r.cache_k])
    hv = torch.stack([dev(head_major(x, 16), dtype) for x in r.cache_v])
    r.do_cow(pairs)
    o.copy_blocks(dk, dv, dev(np.array(pairs, np.int32)), 16)
    assert np.array_equal(to_np(dk), r.cache_k) and np.array_equal(to_np(dv), r.cache_v)
    o.copy_blocks(hk, hv, dev(np.array(pairs, np.int32)), 16)
    for layer in range(3):
        assert np.array_equal(token_major(to_np(hk[layer])), r.cache_k[layer])
        assert np.array_equal(token_major(to_np(hv[layer])), r.cache_v[layer])


def test_rms_norm_and_residual():
    from oracle.model import rms_norm
    o = ops()
    rng = np.random.default_rng(5)
    x = rng.standard_normal((37, 384)).astype(np.float32)
    res = rng.standard_normal((37, 384)).astype(np.float32)
    w = rng.standard_normal(384).astype(np.float32)
    out = torch.empty(37, 384, device="cuda")
    dres = dev(res)
    o.rms_norm(out, dev(x), dev(w), 1e-5, residual=dres)
    np.testing.assert_array_equal(to_np(dres), res + x)
    np.testing.assert_allclose(to_np(out), rms_norm(res + x, w), rtol=2e-6, atol=1e-6)


def test_silu_mul():
    from oracle.model import silu
    o = ops()
    rng = np.random.default_rng(6)
    gu = (rng.standard_normal((19, 2 * 1024)) * 4).astype(np.float32)
    out = torch.empty(19, 1024, device="cuda")
    o.silu_mul(out, dev(gu))
    np.testing.assert_allclose(to_np(out), silu(gu[:, :1024]) * gu[:, 1024:], rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("layout", ["token", "head"])
def test_rope_and_cache_matches_oracle(layout):
    from oracle.attention import apply_rope, build_rope
    o = ops()
    rng = np.random.default_rng(7)
    T, H, Hkv, D = 29, 8, 4, 48
    qkv = rng.standard_normal((T, (H + 2 * Hkv) * D)).astype(np.float32)
    pos = rng.integers(0, 512, size=T).astype(np.int32)
    slots = rng.permutation(304)[:T].astype(np.int32)
    cos, sin = build_rope(D, 512)
    shape = (19, Hkv, 16, D) if layout == "head" else (304, Hkv, D)
    kc = torch.zeros(shape, device="cuda")
    vc = torch.zeros(shape, device="cuda")
    qo = torch.empty(T, H, D, device="cuda")
    o.rope_and_cache(dev(qkv), qo, kc, vc, dev(pos), dev(slots), dev(cos), dev(sin), H, Hkv, D)
    if layout == "head":
        kc, vc = (torch.from_numpy(token_major(to_np(x))) for x in (kc, vc))
    q = qkv[:, :H * D].reshape(T, H, D)
    k = qkv[:, H * D:(H + Hkv) * D].reshape(T, Hkv, D)
    v = qkv[:, (H + Hkv) * D:].reshape(T, Hkv, D)
    np.testing.assert_array_equal(to_np(qo), apply_rope(q, pos, cos, sin))
    np.testing.assert_array_equal(to_np(kc)[slots], apply_rope(k, pos, cos, sin))
    np.testing.assert_array_equal(to_np(vc)[slots], v)


def test_argmax_rows_numpy_ties_and_nan():
    o = ops()
    rng = np.random.default_rng(8)
    x = rng.standard_normal((64, 32000)).astype(np.float32)
    x[3, [5, 900, 31999]] = 50.0            # tie -> lowest index
    x[4, [7, 8]] = np.nan                    # first NaN wins
    x[5, :] = -np.inf
    x[6, -1] = 1e30
    out = torch.empty(64, dtype=torch.int32, device="cuda")
    host = torch.full((70,), -7, dtype=torch.int32, pin_memory=True)
    o.argmax_rows(dev(x), out, host_out=host)
    torch.cuda.synchronize()
    want = np.argmax(x, axis=-1).tolist()
    assert to_np(out).astype(np.int64).tolist() == want
    # the pinned copy written by the same launch; entries past the rows untouched
    assert host[:64].tolist() == want and host[64:].tolist() == [-7] * 6


def test_greedy_verify_matches_oracle():
    from oracle.greedy import verify
    o = ops()
    rng = np.random.default_rng(9)
    S, K, V = 64, 4, 32000
    nd = rng.integers(0, K + 1, size=S).astype(np.int32)
    rows = nd + 1
    row_start = np.zeros(S, np.int32)
    row_start[1:] = np.cumsum(rows)[:-1]
    logits = rng.standard_normal((int(rows.sum()), V)).astype(np.float32)
    drafts = np.zeros((S, K), np.int32)
    for s in range(S):
        acc = int(rng.integers(0, nd[s] + 1))
        for r in range(nd[s]):
            best = int(np.argmax(logits[row_start[s] + r]))
            drafts[s, r] = best if r < acc else (best + 1) % V
    out = torch.empty(S, K + 1, dtype=torch.int32, device="cuda")
    nacc = torch.empty(S, dtype=torch.int32, device="cuda")
    o.greedy_verify(dev(logits), dev(row_start), dev(nd), dev(drafts), out, nacc)
    got, got_acc = to_np(out).astype(np.int64), to_np(nacc).astype(np.int64)
    for s in range(S):
        toks, acc = verify(logits[row_start[s]:row_start[s] + rows[s]], list(drafts[s, :nd[s]]))
        assert got_acc[s] == acc
        assert got[s, :len(toks)].tolist() == toks and (got[s, len(toks):] == -1).all()


@pytest.mark.parametrize("V,stride", [(1003, 1003), (1003, 1004), (32000, 32000), (9, 12)])
def test_greedy_verify_edge_rows(V, stride):
    """vl_greedy_verify (each row read in chunks whose argmax keys meet in one
    atomic maximum per row; the sequence's last workgroup writes the picks up
    to the first mismatch) against the oracle's verify: ties to
    the lowest index, NaN rows (the first NaN wins), rows of -inf, a vocab
    that is not a multiple of 4, rows that are not 16-byte aligned (odd
    stride: the scalar path), no drafts, every draft accepted (the bonus
    row), and max_drafts above every sequence's drafts."""
    from oracle.greedy import verify
    o = ops()
    rng = np.random.default_rng(V + stride)
    S, K = 24, 6
    nd = np.array([rng.integers(0, K) for _ in range(S)], np.int32)
    nd[:3] = [0, K - 1, 1]
    rows = nd + 1
    row_start = np.zeros(S, np.int32)
    row_start[1:] = np.cumsum(rows)[:-1]
    R = int(rows.sum())
    buf = np.full((R, stride), 7.0, np.float32)  # the padding past V is never a candidate
    lg = rng.standard_normal((R, V)).astype(np.float32)
    for r in range(R):
        kind = r % 5
        if kind == 1:  # a tie: the lowest index wins
            c = rng.integers(0, V, 2)
            lg[r, c] = lg[r].max() + 1.0
        elif kind == 2:  # NaNs: the first one wins
            c = np.sort(rng.integers(0, V, 2))
            lg[r, c] = np.nan
        elif kind == 3:
            lg[r] = -np.inf
    buf[:, :V] = lg
    drafts = np.zeros((S, K), np.int32)
    for s in range(S):
        acc = nd[s] if s % 3 == 1 else int(rng.integers(0, nd[s] + 1))
        for r in range(nd[s]):
            best = int(np.argmax(lg[row_start[s] + r]))
            drafts[s, r] = best if r < acc else (best + 1) % V
    flat = torch.from_numpy(buf.reshape(-1)).cuda()
    logits = flat.as_strided((R, V), (stride, 1))
    scratch = torch.zeros(S * (K + 1) + S, dtype=torch.int64, device="cuda")
    for _ in range(2):  # the scratch is left zero: a second call needs no clearing
        out = torch.full((S, K + 1), 99, dtype=torch.int32, device="cuda")
        nacc = torch.full((S,), 99, dtype=torch.int32, device="cuda")
        o.greedy_verify(logits, dev(row_start), dev(nd), dev(drafts), out, nacc, scratch=scratch)
        torch.cuda.synchronize()
        assert int(scratch.abs().sum()) == 0
    got, got_acc = to_np(out).astype(np.int64), to_np(nacc).astype(np.int64)
    full = 0
    for s in range(S):
        toks, acc = verify(lg[row_start[s]:row_start[s] + rows[s]], list(drafts[s, :nd[s]]))
        full += acc == nd[s] and nd[s] > 0
        assert got_acc[s] == acc, s
        assert got[s, :len(toks)].tolist() == toks and (got[s, len(toks):] == -1).all(), s
    assert full >= 3


DECODE_CTX = [1, 5, 15, 16, 17, 100, 255, 256, 257, 1000, 4097, 64, 8192]


@pytest.mark.parametrize("layout", ["token", "head"])
@pytest.mark.parametrize("exact_max_q", [True, False])
def test_bandwidth_decode_path_matches_oracle(exact_max_q, layout):
    """bf16 / D 128 / 32 heads over 8 KV heads / block 16: the bandwidth
    kernel, both cache layouts."""
    b = make_batch([(1, c) for c in DECODE_CTX], 32, 8, 128, 16, seed=11)
    got = run_attention(b, "bf16", exact_max_q=exact_max_q, exact_min_q=exact_max_q,
                        layout=layout)
    check(got, expected(b, "bf16"), "bf16")


SHORT_CTX = [1, 5, 63, 64, 65, 255, 256, 257, 700, 2048]


@pytest.mark.parametrize("D,H,Hkv", [(16, 4, 4), (32, 8, 4), (48, 8, 4), (64, 8, 2), (64, 8, 1),
                                     (48, 16, 2)])
@pytest.mark.parametrize("bs", [1, 16])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("layout", ["token", "head"])
def test_short_decode_kernel(D, H, Hkv, bs, dtype, layout):
    """Decodes of at most 2048 tokens with head_dim <= 64: the one-workgroup-
    per-(sequence, KV head) kernel, chosen by the query and context bounds
    (a sequence without a query in the middle), both cache layouts."""
    seqs = [(1, c) for c in SHORT_CTX[:5]] + [(0, 30)] + [(1, c) for c in SHORT_CTX[5:]]
    b = make_batch(seqs, H, Hkv, D, bs, seed=D + H + bs)
    got = run_attention(b, dtype, ctx_hint=True, layout=layout)
    check(got, expected(b, dtype), dtype)


@pytest.mark.parametrize("seqs", [[(1, c) for c in SHORT_CTX],
                                  [(1, 40), (7, 300), (1, 2000), (16, 16), (3, 5000)]])
@pytest.mark.parametrize("ctx_hint", [True, False])
@pytest.mark.parametrize("layout", ["token", "head"])
@pytest.mark.parametrize("D", [48, 128, 80])
def test_fp32_query_over_bf16_cache(seqs, ctx_hint, layout, D):
    """VL_DTYPE_F32_BF16KV: fp32 query and output over bf16 caches (decodes
    by the short-decode kernel when the bounds allow; the rest by the fp32
    MFMA tile kernel, which widens the cache elements when it stages them,
    for head_dims with a tile instantiation (48, 128), else by the generic
    kernel (80); then the combine) against the oracle on the bf16 K/V values,
    at the fp32 tolerance; both cache layouts."""
    o = ops()
    b = make_batch(seqs, 8, 4, D, 16, seed=len(seqs) + ctx_hint + D)
    q = dev(b["q"])
    kc, vc = caches(b, torch.bfloat16, layout)
    S, T = len(seqs), b["q"].shape[0]
    ws = o.AttentionWorkspace().get(o.paged_attention_workspace_size(S, T, 8, D,
                                                                     int(b["seq_lens"].max())))
    out = torch.full_like(q, float("nan"))
    q_lens = np.diff(b["qsl"])
    o.paged_attention(out, q, kc, vc, dev(b["block_tables"]), dev(b["seq_lens"]), dev(b["qsl"]),
                      b["scale"], 16, ws, max_query_len=int(q_lens.max()),
                      max_context_len=int(b["seq_lens"].max()) if ctx_hint else 0)
    want = oracle_attention(b, b["q"], bf16_round(b["k_cache"]), bf16_round(b["v_cache"]))
    check(to_np(out), want, "f32")


@pytest.mark.parametrize("seqs", [[(1, c) for c in SHORT_CTX],
                                  [(1, 40), (7, 300), (1, 2000), (16, 16), (3, 5000)]])
@pytest.mark.parametrize("ctx_hint", [True, False])
@pytest.mark.parametrize("layout", ["token", "head"])
@pytest.mark.parametrize("D", [48, 128, 80])
def test_fp32_query_over_fp8_cache(seqs, ctx_hint, layout, D):
    """VL_DTYPE_F32_FP8KV: fp32 query and output over FP8 E4M3 caches (the
    short-decode kernel when the bounds allow; else the fp32 MFMA tile kernel
    widening the FP8 elements exactly when it stages them (head_dim 48, 128)
    or the generic kernel (80); then the combine) against the oracle on the
    FP8 values of K/V, at the fp32 tolerance; poisoned slots hold the FP8 NaN
    code."""
    from oracle.attention import fp8_e4m3_decode, fp8_e4m3_encode
    o = ops()
    b = make_batch(seqs, 8, 4, D, 16, seed=7 + len(seqs) + ctx_hint + D)
    kq, vq = fp8_e4m3_decode(fp8_e4m3_encode(b["k_cache"])), fp8_e4m3_decode(fp8_e4m3_encode(b["v_cache"]))
    fb = dict(b, k_cache=kq, v_cache=vq)

    def fp8_dev(x):
        return dev(fp8_e4m3_encode(x)).view(torch.float8_e4m3fn)

    if layout == "head":
        kc, vc = fp8_dev(head_major(b["k_cache"], 16)), fp8_dev(head_major(b["v_cache"], 16))
    else:
        kc, vc = fp8_dev(b["k_cache"]), fp8_dev(b["v_cache"])
    q = dev(b["q"])
    S, T = len(seqs), b["q"].shape[0]
    ws = o.AttentionWorkspace().get(o.paged_attention_workspace_size(S, T, 8, D,
                                                                     int(b["seq_lens"].max())))
    out = torch.full_like(q, float("nan"))
    q_lens = np.diff(b["qsl"])
    o.paged_attention(out, q, kc, vc, dev(b["block_tables"]), dev(b["seq_lens"]), dev(b["qsl"]),
                      b["scale"], 16, ws, max_query_len=int(q_lens.max()),
                      max_context_len=int(b["seq_lens"].max()) if ctx_hint else 0)
    check(to_np(out), oracle_attention(fb), "f32")


@pytest.mark.parametrize("layout", ["token", "head"])
def test_fp8_cache_writer_rounds_like_the_oracle(layout):
    """The RoPE + K/V writer into FP8 E4M3 caches stores the oracle's byte for
    every value: rotated k (the fp32 rotation is bit-exact with NumPy's), and
    v rows holding ties between neighbouring FP8 values, values around 448,
    infinities, tiny and subnormal values."""
    from oracle.attention import apply_rope, build_rope, fp8_e4m3_decode, fp8_e4m3_encode
    o = ops()
    rng = np.random.default_rng(9)
    T, H, Hkv, D = 32, 8, 4, 48
    qkv = (rng.standard_normal((T, (H + 2 * Hkv) * D)) * 3).astype(np.float32)
    pos8 = fp8_e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    special = np.concatenate([((pos8[:-1] + pos8[1:]) / 2).astype(np.float32),  # every tie
                              np.array([448, 449, 463.9, 464, 464.1, 1e9, np.inf, 2.0 ** -10,
                                        3 * 2.0 ** -11, 1e-30, 0.0], np.float32)])
    special = np.concatenate([special, -special])
    vpart = qkv[:, (H + Hkv) * D:].reshape(-1)
    vpart[:special.size] = special
    qkv[:, (H + Hkv) * D:] = vpart.reshape(T, Hkv * D)
    pos = rng.integers(0, 512, size=T).astype(np.int32)
    slots = rng.permutation(320)[:T].astype(np.int32)
    cos, sin = build_rope(D, 512)
    shape = (20, Hkv, 16, D) if layout == "head" else (320, Hkv, D)
    kc = torch.zeros(shape, device="cuda", dtype=torch.float8_e4m3fn)
    vc = torch.zeros(shape, device="cuda", dtype=torch.float8_e4m3fn)
    qo = torch.empty(T, H, D, device="cuda")
    o.rope_and_cache(dev(qkv), qo, kc, vc, dev(pos), dev(slots), dev(cos), dev(sin), H, Hkv, D)
    torch.cuda.synchronize()
    kb, vb = (x.view(torch.uint8).cpu().numpy() for x in (kc, vc))
    if layout == "head":
        kb, vb = token_major(kb), token_major(vb)
    k = apply_rope(qkv[:, H * D:(H + Hkv) * D].reshape(T, Hkv, D), pos, cos, sin)
    v = qkv[:, (H + Hkv) * D:].reshape(T, Hkv, D)
    assert np.array_equal(kb[slots], fp8_e4m3_encode(k))
    assert np.array_equal(vb[slots], fp8_e4m3_encode(v))


def test_short_decode_reads_no_plan():
    """The short-decode run reads nothing from the workspace: a run on a
    workspace holding no plan (every byte 0xff) gives the oracle's output."""
    o = ops()
    b = make_batch([(1, c) for c in (40, 2000, 1)], 8, 4, 48, 16, seed=31)
    q, kc, vc = dev(b["q"]), dev(b["k_cache"]), dev(b["v_cache"])
    ws = o.AttentionWorkspace().get(o.paged_attention_workspace_size(3, 3, 8, 48, 2000))
    ws.fill_(255)
    out = torch.full_like(q, float("nan"))
    o.paged_attention_run(out, q, kc, vc, dev(b["block_tables"]), dev(b["seq_lens"]),
                          dev(b["qsl"]), b["scale"], 16, ws, max_query_len=1, min_query_len=1,
                          max_context_len=2000)
    check(to_np(out), expected(b, "f32"), "f32")


def test_bandwidth_decode_chunks_without_split():
    """Workspace with no room for partials: each item loops over 256-token chunks."""
    o = ops()
    b = make_batch([(1, c) for c in (3000, 700, 257, 16)], 32, 8, 128, 16, seed=12)
    got = run_attention(b, "bf16", ws_bytes=o.lib().vl_paged_attention_min_workspace(4))
    check(got, expected(b, "bf16"), "bf16")


def many_sequences(S, seed):
    """S sequences, mostly decodes: a run of equal contexts (one tail-range
    bucket for all of them), contexts of 1..130 keys (split into 64-key
    ranges when the decode tokens are few), and every tenth sequence a
    multi-query chunk of 2..20 queries."""
    rng = np.random.default_rng(seed)
    seqs = [(1, 77)] * (S // 4)
    for i in range(S - len(seqs)):
        if i % 10 == 9:
            q = int(rng.integers(2, 21))
            seqs.append((q, q + int(rng.integers(0, 60))))
        else:
            seqs.append((1, int(rng.integers(1, 131))))
    order = rng.permutation(S)
    return [seqs[i] for i in order]


@pytest.mark.parametrize("small_ws", [False, True])
@pytest.mark.parametrize("S", [300, 1100])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_plans_over_many_sequences(S, dtype, small_ws):
    """The plan with several sequences per plan thread: from registers (300)
    and re-read from memory (1100, above what a plan thread caches); with the
    smallest workspace the plan doubles its range and partition lengths
    until nothing splits."""
    o = ops()
    b = make_batch(many_sequences(S, seed=S), 16, 4, 128, 16, seed=S)
    ws = o.lib().vl_paged_attention_min_workspace(S) if small_ws else None
    check(run_attention(b, dtype, ws_bytes=ws), expected(b, dtype), dtype)


def test_bandwidth_decode_with_16_kv_heads():
    b = make_batch([(1, c) for c in (33, 600)], 64, 16, 128, 16, seed=13)
    check(run_attention(b, "bf16"), expected(b, "bf16"), "bf16")


def test_plan_once_run_per_layer():
    """One plan serves several runs over different caches (one per layer)."""
    o = ops()
    b0 = make_batch([(1, 300), (7, 50), (1, 2000)], 32, 8, 128, 16, seed=20, num_blocks=200)
    ws = o.AttentionWorkspace().get(o.paged_attention_workspace_size(3, 9, 32, 128, 2000))
    bt, sl, qsl = dev(b0["block_tables"]), dev(b0["seq_lens"]), dev(b0["qsl"])
    for layer in range(3):
        rng = np.random.default_rng(100 + layer)
        b = dict(b0)
        b["q"] = rng.standard_normal(b0["q"].shape).astype(np.float32)
        for name in ("k_cache", "v_cache"):
            fresh = rng.standard_normal(b0[name].shape).astype(np.float32)
            b[name] = np.where(np.isnan(b0[name]), np.nan, fresh).astype(np.float32)
        q = dev(b["q"], torch.bfloat16)
        kc, vc = dev(b["k_cache"], torch.bfloat16), dev(b["v_cache"], torch.bfloat16)
        if layer == 0:
            o.paged_attention_plan(q, kc, sl, qsl, 16, ws)
        out = torch.empty_like(q)
        o.paged_attention_run(out, q, kc, vc, bt, sl, qsl, b["scale"], 16, ws, max_query_len=7)
        check(to_np(out), expected(b, "bf16"), "bf16")


# -- MFMA tile path (multi-query rows: chunked prefill, speculative verify) ----
TILE_SHAPES = [("f32", 8, 4, 48), ("f32", 8, 2, 64), ("f32", 4, 4, 16), ("f32", 16, 4, 128),
               ("f32", 4, 1, 32), ("bf16", 32, 8, 128), ("bf16", 8, 2, 64), ("bf16", 6, 3, 128)]


@pytest.mark.parametrize("dtype,H,Hkv,D", TILE_SHAPES)
@pytest.mark.parametrize("bs", [1, 4, 16, 32])
@pytest.mark.parametrize("layout", ["token", "head"])
def test_tile_prefill_chunks_with_prior_context(dtype, H, Hkv, D, bs, layout):
    """Chunks that start mid-block after prior context, causal within the chunk,
    plus decodes and a 1-token context, all in one call. Block sizes cover
    every staging path: per-key block lookups (1), per-quad V lookups (4),
    one block per 16-key K unit (16, 32); the unowned tail slots of a
    sequence's last block are NaN."""
    seqs = [(37, 37), (100, 133), (1, 90), (64, 64 + 200), (17, 500), (3, 3), (2, 40)]
    b = make_batch(seqs, H, Hkv, D, bs, seed=30 + D + bs)
    check(run_attention(b, dtype, layout=layout), expected(b, dtype), dtype)


@pytest.mark.parametrize("layout", ["token", "head"])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_tile_speculative_verify_rows_split_over_long_context(dtype, layout):
    """5 queries per sequence over long contexts: the context is split into
    partitions and merged; also with no room for partials."""
    seqs = [(5, 3000), (5, 1025), (5, 5), (4, 700), (5, 6001)]
    b = make_batch(seqs, 32, 8, 128, 16, seed=40)
    want = expected(b, dtype)
    check(run_attention(b, dtype, layout=layout), want, dtype)
    o = ops()
    check(run_attention(b, dtype, ws_bytes=o.lib().vl_paged_attention_min_workspace(len(seqs)),
                        layout=layout), want, dtype)


def test_tile_fp32_meets_the_reference_tolerance_at_the_tinyllama_shape():
    """fp32, 8 Q heads over 4 KV heads, D 48 (the TinyLlama mix): a 1024-token
    budget of prefill chunks, rtol 1e-4 / atol 1e-5 as the reference's test."""
    seqs = [(256, 256), (251, 251), (200, 300), (17, 480), (100, 100), (1, 77), (1, 512)]
    b = make_batch(seqs, 8, 4, 48, 16, seed=41)
    got = run_attention(b, "f32")
    np.testing.assert_allclose(got, oracle_attention(b), rtol=1e-4, atol=1e-5)


def test_tile_many_rows_per_kv_head():
    """A 512-token chunk: 2048 (token, head) rows per KV head, 32 row blocks."""
    b = make_batch([(512, 512 + 300), (1, 2000)], 32, 8, 128, 16, seed=42)
    check(run_attention(b, "bf16"), expected(b, "bf16"), "bf16")


def test_bandwidth_decode_split_merge_across_repeated_runs():
    """A ragged decode batch (contexts 64..6000, so many sequences are split
    into ranges merged inside the kernel) run 4 times under one plan with
    fresh K/V each time: a merge that read another run's partials, or a
    counter left non-zero, would fail a later run."""
    o = ops()
    rng = np.random.default_rng(50)
    ctxs = [int(c) for c in np.clip(rng.lognormal(np.log(900), 0.8, size=48), 64, 6000)]
    b0 = make_batch([(1, c) for c in ctxs], 32, 8, 128, 16, seed=51)
    S = len(ctxs)
    ws = o.AttentionWorkspace().get(o.paged_attention_workspace_size(S, S, 32, 128, max(ctxs)))
    bt, sl, qsl = dev(b0["block_tables"]), dev(b0["seq_lens"]), dev(b0["qsl"])
    for run in range(4):
        r = np.random.default_rng(200 + run)
        b = dict(b0)
        b["q"] = r.standard_normal(b0["q"].shape).astype(np.float32)
        for name in ("k_cache", "v_cache"):
            fresh = r.standard_normal(b0[name].shape).astype(np.float32)
            b[name] = np.where(np.isnan(b0[name]), np.nan, fresh).astype(np.float32)
        q = dev(b["q"], torch.bfloat16)
        kc, vc = dev(b["k_cache"], torch.bfloat16), dev(b["v_cache"], torch.bfloat16)
        if run == 0:
            o.paged_attention_plan(q, kc, sl, qsl, 16, ws)
        out = torch.empty_like(q)
        o.paged_attention_run(out, q, kc, vc, bt, sl, qsl, b["scale"], 16, ws, max_query_len=1)
        check(to_np(out), expected(b, "bf16"), "bf16")


# -- closed forms at forced multi-partition splits ----------------------------
def _plan_header(ws):
    """The plan's first 16 int32 of the workspace: [2] the tile partition
    length, [3] the split partial rows written, [7] the decode range length."""
    torch.cuda.synchronize()
    return ws[:64].view(torch.int32).cpu().numpy()


def _closed_form_batch(seqs, H, Hkv, D, seed, dominant):
    """Q/K/V of a batch whose exact attention is known without the oracle.
    dominant=False: every key of a KV head is the same vector, so each query
    attends uniformly and its output is the mean of V over its causal keys.
    dominant=True: every query row of KV group g is the same vector u_g and
    one key per sequence (at 0.6 of the context, inside a middle partition)
    is 40 u_g / |u_g|, a score ~40 above the N(0,1) others, so the output is
    that key's V row."""
    b = make_batch(seqs, H, Hkv, D, 16, seed=seed)
    rng = np.random.default_rng(seed + 1)
    rep = H // Hkv
    kc = b["k_cache"]
    q = b["q"]
    star = []
    for i, t in enumerate(b["tables"]):
        ctx = int(b["seq_lens"][i])
        slots = (t[:, None].astype(np.int64) * 16 + np.arange(16)[None, :]).reshape(-1)[:ctx]
        q0, q1 = b["qsl"][i], b["qsl"][i + 1]
        if not dominant:
            kc[slots] = bf16_round(rng.standard_normal((1, Hkv, D)).astype(np.float32))
            star.append(None)
        else:
            u = bf16_round(rng.standard_normal((Hkv, D)).astype(np.float32))
            q[q0:q1] = np.repeat(u, rep, axis=0)[None]
            j = int(0.6 * ctx)
            kc[slots[j]] = bf16_round(40.0 * u / np.linalg.norm(u, axis=1, keepdims=True))
            star.append(j)
    for name in ("q", "k_cache", "v_cache"):
        b[name] = bf16_round(b[name])
    want = np.zeros_like(b["q"])
    for i, t in enumerate(b["tables"]):
        ctx = int(b["seq_lens"][i])
        slots = (t[:, None].astype(np.int64) * 16 + np.arange(16)[None, :]).reshape(-1)[:ctx]
        q0, q1 = b["qsl"][i], b["qsl"][i + 1]
        vv = b["v_cache"][slots].astype(np.float64)              # [ctx, Hkv, D]
        for j in range(q1 - q0):
            pos = ctx - (q1 - q0) + j
            row = vv[star[i]] if dominant else vv[:pos + 1].mean(axis=0)   # [Hkv, D]
            want[q0 + j] = np.repeat(row, rep, axis=0)
    return b, want


@pytest.mark.parametrize("dominant", [False, True])
@pytest.mark.parametrize("q_len", [1, 5])
def test_closed_forms_at_forced_splits(dominant, q_len):
    """Contexts of 32768 and 8192 keys split into many partitions (the header
    of the plan shows partition / range lengths far below the context and
    split rows written), merged by the decode kernel's last arriver (q_len 1)
    or the combine kernel (q_len 5): uniform attention gives the mean of V,
    a dominant key gives its V, every row within 2e-2 normwise."""
    o = ops()
    seqs = [(q_len, 32768), (q_len, 8192), (q_len, 20000)]
    b, want = _closed_form_batch(seqs, 32, 8, 128, 60 + q_len, dominant)
    q = dev(b["q"], torch.bfloat16)
    kc, vc = dev(b["k_cache"], torch.bfloat16), dev(b["v_cache"], torch.bfloat16)
    out = torch.empty_like(q)
    S, T = len(seqs), q.shape[0]
    ws = o.AttentionWorkspace().get(o.paged_attention_workspace_size(S, T, 32, 128, 32768))
    o.paged_attention(out, q, kc, vc, dev(b["block_tables"]), dev(b["seq_lens"]), dev(b["qsl"]),
                      b["scale"], 16, ws, max_query_len=q_len)
    hdr = _plan_header(ws)
    split_len = hdr[7] if q_len == 1 else hdr[2]
    assert hdr[3] > 0 and split_len <= 8192 // 4, f"no forced split: header {hdr[:13]}"
    assert_rows_close(to_np(out), want, BF16_ROW_REL, f"q_len {q_len} dominant {dominant}")


def test_resolve_tokens_takes_previous_step_ids():
    """vl_resolve_tokens: ids t < 0 become prev[-t - 1]; out-of-range
    references become 0; others are kept."""
    o = ops()
    rng = np.random.default_rng(70)
    prev = rng.integers(0, 32000, size=37).astype(np.int32)
    tok = rng.integers(0, 32000, size=300).astype(np.int32)
    refs = rng.choice(300, size=120, replace=False)
    tok[refs] = -1 - rng.integers(0, 37, size=120)
    tok[refs[:3]] = [-38, -1000, -(2 ** 31)]  # past the end of prev
    want = tok.copy()
    neg = want < 0
    idx = -want[neg].astype(np.int64) - 1
    want[neg] = np.where(idx < 37, prev[np.minimum(idx, 36)], 0)
    d = dev(tok)
    o.resolve_tokens(d, dev(prev))
    assert np.array_equal(to_np(d).astype(np.int64), want.astype(np.int64))


@pytest.mark.parametrize("D,q_len", [(48, 1), (128, 2), (80, 2)])
def test_fp8_cache_values_decode_exactly(D, q_len):
    """Every FP8 E4M3 code (NaN and subnormals included) comes out of the
    attention as the oracle's decoded value: with a zero query the first query
    of each sequence sees one key with weight exactly 1, so its output is that
    key's V row decoded (the short-decode kernel at head_dim 48, the fp32
    tile kernel at 128, the generic kernel at 80)."""
    from oracle.attention import fp8_e4m3_decode
    o = ops()
    S = -(-256 // D)
    codes = np.resize(np.arange(256, dtype=np.uint8), S * D).reshape(S, D)
    kc = np.full((S * 16, 1, D), 0x38, np.uint8)  # every key 1.0
    vc = np.full((S * 16, 1, D), 0x38, np.uint8)
    vc[np.arange(S) * 16, 0, :] = codes  # key 0 of sequence s: the codes
    f8 = lambda a: dev(a).view(torch.float8_e4m3fn)
    q = torch.zeros((S * q_len, 1, D), dtype=torch.float32, device="cuda")
    out = torch.full_like(q, 7.0)
    ws = o.AttentionWorkspace().get(o.paged_attention_workspace_size(S, S * q_len, 1, D, q_len))
    o.paged_attention(out, q, f8(kc), f8(vc), dev(np.arange(S, dtype=np.int32).reshape(S, 1)),
                      dev(np.full(S, q_len, np.int32)),
                      dev(np.arange(S + 1, dtype=np.int32) * q_len), 1.0 / np.sqrt(D), 16, ws,
                      max_query_len=q_len, min_query_len=q_len, max_context_len=q_len)
    got = to_np(out).reshape(S, q_len, D)[:, 0, :]
    np.testing.assert_array_equal(got, fp8_e4m3_decode(codes))


@pytest.mark.parametrize("cache", ["f32", "bf16", "fp8"])
@pytest.mark.parametrize("D,H,Hkv,dm", [(48, 8, 4, 384), (16, 4, 2, 64), (64, 8, 1, 512),
                                        (32, 16, 2, 96)])
@pytest.mark.parametrize("layout", ["token", "head"])
def test_decode_attention_wo_equals_attention_then_wo(cache, D, H, Hkv, dm, layout):
    """vl_decode_attention_wo: parts[s, g] = (sequence s's attention outputs of
    KV head g's query heads) @ those rows of wo, and their sum over g is
    attn @ wo (vllmlite/model.py:114), against float64 products of the
    oracle's attention rows (a sequence without a query in the middle keeps
    its parts unwritten)."""
    o = ops()
    seqs = [(1, c) for c in SHORT_CTX[:4]] + [(0, 30)] + [(1, c) for c in SHORT_CTX[4:7]]
    from oracle.attention import fp8_e4m3_decode, fp8_e4m3_encode
    b = make_batch(seqs, H, Hkv, D, 16, seed=D + H + dm)
    if cache == "fp8":
        def fp8_dev(x):
            return dev(fp8_e4m3_encode(x)).view(torch.float8_e4m3fn)
        hm = (lambda x: head_major(x, 16)) if layout == "head" else (lambda x: x)
        kc, vc = fp8_dev(hm(b["k_cache"])), fp8_dev(hm(b["v_cache"]))
        ck = lambda a: fp8_e4m3_decode(fp8_e4m3_encode(a))  # noqa: E731
    else:
        kc, vc = caches(b, torch.float32 if cache == "f32" else torch.bfloat16, layout)
        ck = (lambda a: a) if cache == "f32" else bf16_round
    rng = np.random.default_rng(dm + Hkv)
    wo = (rng.standard_normal((H * D, dm)) / np.sqrt(H * D)).astype(np.float32)
    S = len(seqs)
    parts = torch.full((S, Hkv, dm), float("nan"), device="cuda")
    o.decode_attention_wo(parts, dev(b["q"]), kc, vc, dev(b["block_tables"]), dev(b["seq_lens"]),
                          dev(b["qsl"]), b["scale"], 16, dev(wo), int(b["seq_lens"].max()))
    torch.cuda.synchronize()
    att = oracle_attention(b, b["q"], ck(b["k_cache"]), ck(b["v_cache"])).astype(np.float64)
    got = parts.cpu().numpy().astype(np.float64)
    rep = H // Hkv
    for i, (q, _) in enumerate(seqs):
        if q == 0:
            assert np.isnan(got[i]).all()
            continue
        t = b["qsl"][i]
        for g in range(Hkv):
            rows = att[t, g * rep:(g + 1) * rep].reshape(-1)
            want = rows @ wo[g * rep * D:(g + 1) * rep * D].astype(np.float64)
            err = np.abs(got[i, g] - want).max() / max(1e-3, np.abs(want).max())
            assert err < 2e-5, (i, g, err)
        total = att[t].reshape(-1) @ wo.astype(np.float64)
        np.testing.assert_allclose(got[i].sum(0), total, rtol=0, atol=2e-5 * np.abs(total).max())


@pytest.mark.parametrize("D,H,Hkv,dm", [(48, 8, 4, 384), (64, 8, 1, 512)])
def test_decode_attention_wo_same_bits_for_any_column_split(D, H, Hkv, dm):
    """A batch of few (sequence, KV head) items splits each item's wo columns
    over 4 workgroups, a large batch keeps them in one; the column sums are
    ((S0 + S1) + S2) + S3 over the same k quarters either way, so the first 8
    sequences' parts are the same bits alone (32 items or 8) as within 72."""
    o = ops()
    rng = np.random.default_rng(D + dm)
    seqs = [(1, int(c)) for c in rng.integers(1, 400, 72)]
    b = make_batch(seqs, H, Hkv, D, 16, seed=dm)
    kc, vc = caches(b, torch.float32)
    wo = dev((rng.standard_normal((H * D, dm)) / np.sqrt(H * D)).astype(np.float32))
    q, bt, lens, qsl = dev(b["q"]), dev(b["block_tables"]), dev(b["seq_lens"]), dev(b["qsl"])
    big = torch.full((72, Hkv, dm), float("nan"), device="cuda")
    o.decode_attention_wo(big, q, kc, vc, bt, lens, qsl, b["scale"], 16, wo, 400)
    small = torch.full((8, Hkv, dm), float("nan"), device="cuda")
    o.decode_attention_wo(small, q, kc, vc, bt[:8], lens[:8], qsl[:9], b["scale"], 16, wo, 400)
    torch.cuda.synchronize()
    assert torch.isfinite(big).all()
    assert torch.equal(big[:8], small)


def test_decode_attention_wo_refuses_other_batches():
    o = ops()
    b = make_batch([(1, 40), (1, 3000)], 8, 4, 48, 16, seed=3)
    parts = torch.zeros((2, 4, 384), device="cuda")
    wo = torch.zeros((384, 384), device="cuda")
    with pytest.raises(RuntimeError):  # a context beyond the short-decode bound
        o.decode_attention_wo(parts, dev(b["q"]), dev(b["k_cache"]), dev(b["v_cache"]),
                              dev(b["block_tables"]), dev(b["seq_lens"]), dev(b["qsl"]),
                              b["scale"], 16, wo, 3000)


@pytest.mark.parametrize("dtype,D,decode", [("bf16", 128, False), ("bf16", 128, True),
                                             ("f32", 48, True)])
def test_split_rows_merged_in_kernel_over_repeated_runs(dtype, D, decode):
    """Short-query sequences over long contexts split into partitions that the
    kernel running them merges itself (the row block's last workgroup; no
    combine launch): one plan, then four runs as a model's layers run them.
    Every run gives the same bits and matches the oracle, so the arrival
    counters and the queue counters are back at zero after each run; the mix
    of lengths puts short last partitions behind full ones (the bf16
    longest-first order) and sequences that are not split beside split ones.
    bf16 with a decode among them runs in the one-launch step kernel, without
    in the tile kernel; fp32 in the fp32 tile kernel."""
    o = ops()
    seqs = [(5, 9000), (5, 300), (3, 20000), (16, 5000), (5, 64), (2, 12345), (5, 4097)]
    if decode:
        seqs.insert(3, (1, 7000))
    H, Hkv = (32, 8) if dtype == "bf16" else (8, 4)
    b = make_batch(seqs, H, Hkv, D, 16, seed=D + 3)
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    q = dev(b["q"], tdt)
    kc, vc = caches(b, tdt, "token")
    S, T = len(seqs), b["q"].shape[0]
    ws = o.AttentionWorkspace().get(o.paged_attention_workspace_size(S, T, H, D,
                                                                     int(b["seq_lens"].max())))
    bt, lens, qsl = dev(b["block_tables"]), dev(b["seq_lens"]), dev(b["qsl"])
    o.paged_attention_plan(q, kc, lens, qsl, 16, ws)
    outs = []
    for _ in range(4):
        out = torch.full_like(q, float("nan"))
        o.paged_attention_run(out, q, kc, vc, bt, lens, qsl, b["scale"], 16, ws,
                              max_query_len=16, min_query_len=1 if decode else 2)
        outs.append(to_np(out))
    want = expected(b, dtype)
    for got in outs:
        assert np.array_equal(got.view(np.uint8), outs[0].view(np.uint8))
        check(got, want, dtype)

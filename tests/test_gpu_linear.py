"""vl_linear_rows (K6): the TinyLlama projections (16-row tiles; one tile for
a decode step's <= 16 rows, several for a prefill step's, up to 4 of them one
after another in a workgroup when the grid is large) with RMSNorm /
residual / SwiGLU fused, against float64 NumPy of the reference's
formulas (vllmlite/model.py:17-23, 96-101, 114-120): rms_norm(x, w) =
x / sqrt(mean(x^2) + 1e-5) * w, silu(x) = x / (1 + exp(-x))."""

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _ops():
    from vllmlite_amd import ops
    return ops


def _rms(x, w, eps=1e-5):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _close(got, want, tol=2e-5):
    scale = max(1.0, float(np.abs(want).max()))
    np.testing.assert_allclose(got, want, rtol=0, atol=tol * scale)


@pytest.mark.parametrize("rows", [1, 7, 16, 17, 100, 1000, 1024])
@pytest.mark.parametrize("k,n", [(384, 1152), (384, 384), (384, 261), (1024, 384), (64, 192),
                                 (128, 64), (496, 40)])
@pytest.mark.parametrize("norm", [False, True])
def test_store_and_accumulate(rows, k, n, norm):
    o = _ops()
    rng = np.random.default_rng(rows * 1000 + k + n + norm)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    w = (0.02 * rng.standard_normal((k, n))).astype(np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    res = rng.standard_normal((rows, n)).astype(np.float32)
    xin = _rms(x.astype(np.float64), g.astype(np.float64)) if norm else x.astype(np.float64)
    want = xin @ w.astype(np.float64)
    dx, dw, dg = (torch.from_numpy(a).cuda() for a in (x, w, g))
    out = torch.full((rows, n), float("nan"), device="cuda")
    o.linear_rows(out, dx, dw, dg if norm else None, mode=o.LINEAR_STORE)
    acc = torch.from_numpy(res).cuda()
    o.linear_rows(acc, dx, dw, dg if norm else None, mode=o.LINEAR_ACCUMULATE)
    torch.cuda.synchronize()
    _close(out.cpu().numpy(), want)
    _close(acc.cpu().numpy(), res + want)


@pytest.mark.parametrize("rows", [1, 16, 33, 1000])
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("k,dff", [(384, 1024), (64, 128)])
def test_swiglu(rows, norm, k, dff):
    """w_gate | w_up side by side ([k, 2 d_ff]): out = silu(h @ w_gate) *
    (h @ w_up); k shorter than the unrolled depth too."""
    o = _ops()
    rng = np.random.default_rng(7 + rows + norm + k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    w = (0.05 * rng.standard_normal((k, 2 * dff))).astype(np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    h = _rms(x.astype(np.float64), g.astype(np.float64)) if norm else x.astype(np.float64)
    w64 = w.astype(np.float64)
    want = _silu(h @ w64[:, :dff]) * (h @ w64[:, dff:])
    out = torch.full((rows, dff), float("nan"), device="cuda")
    o.linear_rows(out, torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(),
                  torch.from_numpy(g).cuda() if norm else None, mode=o.LINEAR_SWIGLU)
    torch.cuda.synchronize()
    _close(out.cpu().numpy(), want)


@pytest.mark.parametrize("k", [384, 1024, 48])
def test_norm_as_row_scale_matches_rms_norm_kernel(k):
    """The fused RMSNorm is applied as ((x * g) @ W) / rms(x): with an identity
    weight the projection returns (x * g) / rms, which differs from
    vl_rms_norm's (x / rms) * g by the order of two roundings only (a few
    ulps), and the scale is exactly 1 / rms of the row's own elements."""
    o = _ops()
    rng = np.random.default_rng(3 + k)
    x = torch.from_numpy(rng.standard_normal((16, k)).astype(np.float32)).cuda()
    g = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)).cuda()
    eye = torch.eye(k, device="cuda")
    got = torch.empty((16, k), device="cuda")
    o.linear_rows(got, x, eye, g, mode=o.LINEAR_STORE)
    ref = torch.empty_like(x)
    o.rms_norm(ref, x, g)
    torch.cuda.synchronize()
    np.testing.assert_allclose(got.cpu().numpy(), ref.cpu().numpy(), rtol=4e-7, atol=0)


def test_bad_arguments_raise():
    o = _ops()
    x = torch.zeros((17, 384), device="cuda")
    w = torch.zeros((384, 384), device="cuda")
    out = torch.zeros((17, 384), device="cuda")
    # more rows than 65535 row tiles: refused before any launch
    rc = o.lib().vl_linear_rows(o._ptr(out), 384, o._ptr(x), 384, None, o._ptr(w), 384, None,
                                1e-5, o.LINEAR_ROWS_MAX + 1, 384, 384, o.LINEAR_STORE, o._stream())
    assert rc != 0
    with pytest.raises(RuntimeError):
        o.linear_rows(torch.zeros((4, 384), device="cuda"), torch.zeros((4, 100), device="cuda"),
                      torch.zeros((100, 384), device="cuda"))


@pytest.mark.parametrize("layout", ["token", "head"])
@pytest.mark.parametrize("rows", [1, 13, 16, 37, 700])
@pytest.mark.parametrize("shape", [(8, 4, 48, 384), (4, 2, 16, 64)])
def test_qkv_rope_cache_equals_projection_then_rope(rows, shape, layout):
    """vl_qkv_rope_cache gives the same bits as vl_linear_rows followed by
    vl_rope_and_cache: rotated q, rotated k and v at each row's slot, rows
    with slot -1 writing q only; with head-major caches (8-slot blocks) both
    writers put the same rows there."""
    o = _ops()
    H, Hkv, D, k = shape
    n = (H + 2 * Hkv) * D
    rng = np.random.default_rng(rows + D)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    x = dev(rng.standard_normal((rows, k)).astype(np.float32))
    w = dev((0.05 * rng.standard_normal((k, n))).astype(np.float32))
    g = dev((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32))
    pos = dev(rng.integers(0, 64, rows).astype(np.int32))
    nslots = 40 if rows <= 40 else (rows + 7) // 8 * 8
    slots = rng.permutation(nslots)[:rows].astype(np.int32)
    slots[::5] = -1
    slot = dev(slots)
    ang = rng.standard_normal((64, D // 2)).astype(np.float32)
    cos, sin = dev(np.cos(ang)), dev(np.sin(ang))
    shape = (nslots // 8, Hkv, 8, D) if layout == "head" else (nslots, Hkv, D)
    kc1, vc1 = (torch.full(shape, float("nan"), device="cuda") for _ in range(2))
    kc2, vc2 = kc1.clone(), vc1.clone()
    q1 = torch.empty((rows, H, D), device="cuda")
    q2 = torch.empty_like(q1)
    qkv = torch.empty((rows, n), device="cuda")
    o.linear_rows(qkv, x, w, g, mode=o.LINEAR_STORE)
    o.rope_and_cache(qkv, q1, kc1, vc1, pos, slot, cos, sin, H, Hkv, D)
    o.qkv_rope_cache(q2.view(rows, -1), kc2, vc2, x, w, g, pos, slot, cos, sin, H, Hkv, D)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2)
    assert torch.equal(kc1.nan_to_num(7.0), kc2.nan_to_num(7.0))
    assert torch.equal(vc1.nan_to_num(7.0), vc2.nan_to_num(7.0))
    if layout == "head":  # row (slot, h) of the head-major cache is rotated k / v of slot's row
        from oracle.attention import apply_rope
        kh = kc1.permute(0, 2, 1, 3).reshape(nslots, Hkv, D).cpu().numpy()
        vh = vc1.permute(0, 2, 1, 3).reshape(nslots, Hkv, D).cpu().numpy()
        ok = slots >= 0
        qkvn = qkv.cpu().numpy()
        k_rows = qkvn[:, H * D:(H + Hkv) * D].reshape(rows, Hkv, D)
        want_k = apply_rope(k_rows, pos.cpu().numpy(), cos.cpu().numpy(), sin.cpu().numpy())
        np.testing.assert_array_equal(kh[slots[ok]], want_k[ok])
        np.testing.assert_array_equal(vh[slots[ok]], qkvn[ok, (H + Hkv) * D:].reshape(-1, Hkv, D))


@pytest.mark.parametrize("cdt", ["bf16", "fp8"])
@pytest.mark.parametrize("rows", [1, 16])
def test_qkv_rope_cache_narrow_cache_is_the_rounded_fp32_cache(rows, cdt):
    """With bf16 or FP8 E4M3 caches both K/V writers (vl_qkv_rope_cache and
    vl_rope_and_cache) store exactly the fp32 values rounded to nearest even
    (FP8 saturating), and q (fp32) is unchanged."""
    from oracle.attention import round_bf16, round_fp8_e4m3
    narrow = torch.bfloat16 if cdt == "bf16" else torch.float8_e4m3fn
    rnd = round_bf16 if cdt == "bf16" else round_fp8_e4m3
    o = _ops()
    H, Hkv, D, k = 8, 4, 48, 384
    n = (H + 2 * Hkv) * D
    rng = np.random.default_rng(40 + rows)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    x = dev(rng.standard_normal((rows, k)).astype(np.float32))
    w = dev((0.05 * rng.standard_normal((k, n))).astype(np.float32))
    g = dev((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32))
    pos = dev(rng.integers(0, 64, rows).astype(np.int32))
    slot = dev(rng.permutation(40)[:rows].astype(np.int32))
    ang = rng.standard_normal((64, D // 2)).astype(np.float32)
    cos, sin = dev(np.cos(ang)), dev(np.sin(ang))
    kf, vf = (torch.zeros((40, Hkv, D), device="cuda") for _ in range(2))
    kb, vb, kb2, vb2 = (torch.zeros((40, Hkv, D), device="cuda", dtype=narrow)
                        for _ in range(4))
    qf, qb, qb2 = (torch.empty((rows, H * D), device="cuda") for _ in range(3))
    o.qkv_rope_cache(qf, kf, vf, x, w, g, pos, slot, cos, sin, H, Hkv, D)
    o.qkv_rope_cache(qb, kb, vb, x, w, g, pos, slot, cos, sin, H, Hkv, D)
    qkv = torch.empty((rows, n), device="cuda")
    o.linear_rows(qkv, x, w, g, mode=o.LINEAR_STORE)
    o.rope_and_cache(qkv, qb2.view(rows, H, D), kb2, vb2, pos, slot, cos, sin, H, Hkv, D)
    torch.cuda.synchronize()
    assert torch.equal(qf, qb) and torch.equal(qf, qb2)
    for f32, b16, b16b in ((kf, kb, kb2), (vf, vb, vb2)):
        want = rnd(f32.cpu().numpy())
        assert np.array_equal(b16.float().cpu().numpy(), want)
        assert np.array_equal(b16b.float().cpu().numpy(), want)


@pytest.mark.parametrize("nrows", [9, 1000])
def test_row_index_gathers_input_rows(nrows):
    """With row_index the input rows are x[row_index] (the logits-row gather,
    vllmlite/runner.py:90): the same bits as gathering first."""
    o = _ops()
    rng = np.random.default_rng(11)
    x = torch.from_numpy(rng.standard_normal((40, 384)).astype(np.float32)).cuda()
    w = torch.from_numpy((0.05 * rng.standard_normal((384, 261))).astype(np.float32)).cuda()
    g = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(384)).astype(np.float32)).cuda()
    idx = torch.from_numpy(rng.integers(0, 40, nrows).astype(np.int32)).cuda()
    got = torch.empty((nrows, 261), device="cuda")
    o.linear_rows(got, x, w, g, mode=o.LINEAR_STORE, row_index=idx)
    want = torch.empty_like(got)
    o.linear_rows(want, x[idx.long()].contiguous(), w, g, mode=o.LINEAR_STORE)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_qkv_rope_cache_embedding_gather_and_residual_copy():
    """Layer 0 reads its rows straight from the embedding table
    (tok_emb[token_ids], vllmlite/model.py:93) and writes them out as the
    residual stream: the same bits as gathering first, and x_out equal to
    the gathered rows."""
    o = _ops()
    H, Hkv, D, k, rows = 8, 4, 48, 384, 11
    n = (H + 2 * Hkv) * D
    rng = np.random.default_rng(12)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    table = dev(rng.standard_normal((50, k)).astype(np.float32))
    ids = dev(rng.integers(0, 50, rows).astype(np.int32))
    w = dev((0.05 * rng.standard_normal((k, n))).astype(np.float32))
    g = dev((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32))
    pos = dev(rng.integers(0, 64, rows).astype(np.int32))
    slot = dev(rng.permutation(30)[:rows].astype(np.int32))
    ang = rng.standard_normal((64, D // 2)).astype(np.float32)
    cos, sin = dev(np.cos(ang)), dev(np.sin(ang))
    kc1, vc1 = (torch.zeros((30, Hkv, D), device="cuda") for _ in range(2))
    kc2, vc2 = kc1.clone(), vc1.clone()
    q1 = torch.empty((rows, H * D), device="cuda")
    q2 = torch.empty_like(q1)
    x_out = torch.full((rows, k), float("nan"), device="cuda")
    o.qkv_rope_cache(q1, kc1, vc1, table[ids.long()].contiguous(), w, g, pos, slot, cos, sin, H,
                     Hkv, D)
    o.qkv_rope_cache(q2, kc2, vc2, table, w, g, pos, slot, cos, sin, H, Hkv, D, row_index=ids,
                     x_out=x_out)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    assert torch.equal(x_out, table[ids.long()])


def test_qkv_rope_cache_resolves_placeholder_tokens():
    """A token id -(1 + i) < 0 in row_index stands for prev_ids[i] (the id the
    previous step chose for its row i; 0 when i >= num_prev), as
    vl_resolve_tokens would replace it first: the same bits as resolving on
    the device and then gathering."""
    o = _ops()
    H, Hkv, D, k, rows = 8, 4, 48, 384, 16
    n = (H + 2 * Hkv) * D
    rng = np.random.default_rng(31)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    table = dev(rng.standard_normal((261, k)).astype(np.float32))
    prev = dev(rng.integers(0, 261, 12).astype(np.int32))
    ids_np = rng.integers(0, 261, rows).astype(np.int32)
    ids_np[[0, 3, 4, 9, 15]] = [-1, -12, -5, -13, -40]  # -13, -40: past num_prev -> id 0
    ids = dev(ids_np)
    w = dev(o.tile16(torch.from_numpy((0.05 * rng.standard_normal((k, n))).astype(np.float32)))
            .numpy())
    g = dev(np.ones(k, np.float32))
    pos = dev(rng.integers(0, 64, rows).astype(np.int32))
    slot = dev(rng.permutation(40)[:rows].astype(np.int32))
    ang = rng.standard_normal((64, D // 2)).astype(np.float32)
    cos, sin = dev(np.cos(ang)), dev(np.sin(ang))
    kc1, vc1 = (torch.zeros((40, Hkv, D), device="cuda") for _ in range(2))
    kc2, vc2 = kc1.clone(), vc1.clone()
    q1 = torch.empty((rows, H * D), device="cuda")
    q2 = torch.empty_like(q1)
    x1 = torch.full((rows, k), float("nan"), device="cuda")
    x2 = torch.full((rows, k), float("nan"), device="cuda")
    o.qkv_rope_cache(q1, kc1, vc1, table, w, g, pos, slot, cos, sin, H, Hkv, D, row_index=ids,
                     x_out=x1, prev_ids=prev)
    resolved = ids.clone()
    o.resolve_tokens(resolved, prev)
    o.qkv_rope_cache(q2, kc2, vc2, table, w, g, pos, slot, cos, sin, H, Hkv, D,
                     row_index=resolved, x_out=x2)
    torch.cuda.synchronize()
    want_ids = np.where(ids_np >= 0, ids_np, 0)
    p = prev.cpu().numpy()
    for r, t in enumerate(ids_np):
        if t < 0 and -t - 1 < 12:
            want_ids[r] = p[-t - 1]
    assert np.array_equal(resolved.cpu().numpy(), want_ids)
    assert torch.equal(q1, q2) and torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    assert torch.equal(x1, table[torch.from_numpy(want_ids).long().cuda()])
    assert torch.equal(ids.cpu(), torch.from_numpy(ids_np))  # row_index is only read


@pytest.mark.parametrize("rows", [1, 16])
@pytest.mark.parametrize("k,n", [(384, 1152), (384, 261), (1024, 384), (64, 40)])
@pytest.mark.parametrize("mode", ["store", "accumulate", "swiglu"])
def test_tiled_weights_same_bits(rows, k, n, mode):
    """Weights in 16-column tiles ([ceil(n/16), k, 16], zero past n; SwiGLU:
    gate tiles then up tiles) give the same bits as the row-major weight."""
    o = _ops()
    m = {"store": o.LINEAR_STORE, "accumulate": o.LINEAR_ACCUMULATE, "swiglu": o.LINEAR_SWIGLU}[mode]
    halves = 2 if mode == "swiglu" else 1
    rng = np.random.default_rng(rows + k + n + halves)
    x = torch.from_numpy(rng.standard_normal((rows, k)).astype(np.float32)).cuda()
    w = torch.from_numpy((0.05 * rng.standard_normal((k, halves * n))).astype(np.float32)).cuda()
    g = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)).cuda()
    wt = o.tile16(w, halves)
    assert wt.shape == (halves * -(-n // 16), k, 16)
    init = torch.from_numpy(rng.standard_normal((rows, n)).astype(np.float32)).cuda()
    a, b = init.clone(), init.clone()
    o.linear_rows(a, x, w, g, mode=m)
    o.linear_rows(b, x, wt, g, mode=m)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_qkv_rope_cache_tiled_weights_same_bits():
    o = _ops()
    H, Hkv, D, k, rows = 8, 4, 48, 384, 13
    n = (H + 2 * Hkv) * D
    rng = np.random.default_rng(21)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    x = dev(rng.standard_normal((rows, k)).astype(np.float32))
    w = dev((0.05 * rng.standard_normal((k, n))).astype(np.float32))
    g = dev((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32))
    pos = dev(rng.integers(0, 64, rows).astype(np.int32))
    slot = dev(rng.permutation(30)[:rows].astype(np.int32))
    ang = rng.standard_normal((64, D // 2)).astype(np.float32)
    cos, sin = dev(np.cos(ang)), dev(np.sin(ang))
    kc1, vc1 = (torch.zeros((30, Hkv, D), device="cuda") for _ in range(2))
    kc2, vc2 = kc1.clone(), vc1.clone()
    q1 = torch.empty((rows, H * D), device="cuda")
    q2 = torch.empty_like(q1)
    o.qkv_rope_cache(q1, kc1, vc1, x, w, g, pos, slot, cos, sin, H, Hkv, D)
    o.qkv_rope_cache(q2, kc2, vc2, x, o.tile16(w), g, pos, slot, cos, sin, H, Hkv, D)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(kc1, kc2) and torch.equal(vc1, vc2)


@pytest.mark.parametrize("rows", [1, 4, 7, 16, 33])
@pytest.mark.parametrize("k,n,P", [(384, 1024, 4), (512, 256, 8), (64, 128, 1), (128, 48, 2)])
@pytest.mark.parametrize("norm", [False, True])
def test_linear_rows_parts_equals_summed_input(rows, k, n, P, norm):
    """vl_linear_rows_parts: the SwiGLU projection of x + parts[:, 0] + ... +
    parts[:, P - 1] (summed in that order) gives the same bits as
    vl_linear_rows over the rows summed beforehand in that order, and x_out
    receives those summed rows."""
    o = _ops()
    rng = np.random.default_rng(rows * 31 + k + P + norm)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    parts = (0.3 * rng.standard_normal((rows, P, k))).astype(np.float32)
    w = (0.05 * rng.standard_normal((k, 2 * n))).astype(np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    summed = x.copy()
    for p in range(P):
        summed = summed + parts[:, p]
    wt = o.tile16(torch.from_numpy(w), 2).cuda()
    dx, dp, dg = (torch.from_numpy(a).cuda() for a in (x, parts, g))
    got = torch.full((rows, n), float("nan"), device="cuda")
    x_out = torch.full((rows, k), float("nan"), device="cuda")
    o.linear_rows_parts(got, dx, dp, wt, dg if norm else None, x_out=x_out)
    want = torch.full((rows, n), float("nan"), device="cuda")
    o.linear_rows(want, torch.from_numpy(summed).cuda(), wt, dg if norm else None,
                  mode=o.LINEAR_SWIGLU)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert np.array_equal(x_out.cpu().numpy(), summed)


def _argmax_call(o, x, wt, g, rows, n, scratch, row_index=None, host=None):
    out = torch.full((rows, n), float("nan"), device="cuda")
    ids = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
    o.linear_rows_argmax(out, x, wt, g, ids, scratch, host_ids=host, row_index=row_index)
    return out, ids


@pytest.mark.parametrize("rows", [1, 5, 16, 17, 48, 300])
@pytest.mark.parametrize("k,n", [(384, 261), (1024, 384), (64, 40)])
def test_linear_rows_argmax_is_store_then_argmax(rows, k, n):
    """vl_linear_rows_argmax: the logits of vl_linear_rows (same bits) and each
    row's argmax over them from the same launch, exactly np.argmax's, in the
    device ids and the pinned host copy; the scratch is zero again after every
    call, so calls in a row need no clearing."""
    o = _ops()
    rng = np.random.default_rng(rows + k + n)
    scratch = torch.zeros(rows + 1, dtype=torch.int64, device="cuda")
    host = torch.full((rows,), -1, dtype=torch.int32, pin_memory=True)
    g = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)).cuda()
    for it in range(3):
        src = torch.from_numpy(rng.standard_normal((rows + 9, k)).astype(np.float32)).cuda()
        w = torch.from_numpy((0.05 * rng.standard_normal((k, n))).astype(np.float32)).cuda()
        lidx = torch.from_numpy(rng.integers(0, rows + 9, rows).astype(np.int32)).cuda()
        want = torch.full((rows, n), float("nan"), device="cuda")
        o.linear_rows(want, src, w, g, mode=o.LINEAR_STORE, row_index=lidx)
        out, ids = _argmax_call(o, src, o.tile16(w, 1), g, rows, n, scratch, lidx, host)
        torch.cuda.synchronize()
        assert torch.equal(out, want), it
        want_ids = np.argmax(out.cpu().numpy(), axis=1)
        assert np.array_equal(ids.cpu().numpy(), want_ids), it
        assert np.array_equal(host.numpy(), want_ids), it
        assert int(scratch.abs().sum()) == 0, it


def test_linear_rows_argmax_ties_nan_and_infinities():
    """numpy's rule on crafted rows: x = e_0 (no norm) and a weight that is
    zero but for row 0 make logit c = w[0, c]. Equal maxima go to the lowest
    column, a NaN beats +inf (the first NaN wins), +inf beats every number,
    and a row of -inf gives column 0; the 100 columns span 7 tiles (7
    workgroups fold into each row's key)."""
    o = _ops()
    n, k = 100, 64
    patterns = [
        ({3: 5.0, 40: 5.0, 90: 5.0}, 3),            # a tie across tiles
        ({70: 2.0, 20: 2.0, 21: 2.0}, 20),
        ({10: np.inf, 80: np.nan, 95: np.nan}, 80),  # the first NaN
        ({55: np.inf, 60: 1e38, 99: np.inf}, 55),    # the first +inf
        ("neg_inf", 0),                               # every logit -inf
        ({0: -1.0, 99: -0.5}, 99),                   # the others -3
    ]
    scratch = torch.zeros(2, dtype=torch.int64, device="cuda")
    x = np.zeros((1, k), np.float32)
    x[0, 0] = 1.0
    for spec, want in patterns:
        w = np.zeros((k, n), np.float32)
        if spec == "neg_inf":
            w[0] = -np.inf
        else:
            w[0] = -3.0
            for c, v in spec.items():
                w[0, c] = v
        assert int(np.argmax(w[0])) == want  # the rule the test states is numpy's
        out, ids = _argmax_call(o, torch.from_numpy(x).cuda(),
                                o.tile16(torch.from_numpy(w).cuda(), 1), None, 1, n, scratch)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy()[0], w[0])  # logit c = w[0, c]
        assert int(ids.cpu()[0]) == want, spec
        assert int(scratch.abs().sum()) == 0


def test_linear_rows_argmax_bad_arguments_raise():
    o = _ops()
    x = torch.zeros((4, 64), device="cuda")
    wt = o.tile16(torch.zeros((64, 40), device="cuda"), 1)
    out = torch.zeros((4, 40), device="cuda")
    ids = torch.zeros(4, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError):  # scratch too small (needs rows + 1 words)
        o.linear_rows_argmax(out, x, wt, None, ids, torch.zeros(4, dtype=torch.int64, device="cuda"))
    with pytest.raises(ValueError):  # row-major weight (refused before the call)
        o.linear_rows_argmax(out, x, torch.zeros((64, 40), device="cuda"), None, ids,
                             torch.zeros(5, dtype=torch.int64, device="cuda"))


@pytest.mark.parametrize("rows,extra", [(16, 700), (5, 0), (1, 100_000)])
def test_qkv_rope_cache_reads_and_copies_a_pinned_record(rows, extra):
    """vl_qkv_rope_cache with a record: its token / position / slot indices
    read from pinned host memory (views of the record) give the same bits as
    the same indices on the device, and the launch copies the whole record to
    the device (a record longer than the launch's threads too: 100K words
    against one row's 48 x 512)."""
    o = _ops()
    H, Hkv, D, k = 8, 4, 48, 384
    n = (H + 2 * Hkv) * D
    rng = np.random.default_rng(rows + extra)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    table = dev(rng.standard_normal((261, k)).astype(np.float32))
    prev = dev(rng.integers(0, 261, 12).astype(np.int32))
    w = dev(o.tile16(torch.from_numpy((0.05 * rng.standard_normal((k, n))).astype(np.float32)))
            .numpy())
    g = dev((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32))
    ang = rng.standard_normal((64, D // 2)).astype(np.float32)
    cos, sin = dev(np.cos(ang)), dev(np.sin(ang))
    # the record: tokens (some placeholders), positions, slots, then other words
    toks = rng.integers(0, 261, rows).astype(np.int32)
    toks[::3] = -1 - rng.integers(0, 12, len(toks[::3]))
    rec = np.concatenate([toks, rng.integers(0, 64, rows).astype(np.int32),
                          rng.permutation(40)[:rows].astype(np.int32),
                          rng.integers(-5, 5, extra).astype(np.int32)])
    host = torch.from_numpy(rec).pin_memory()
    drec = dev(rec)
    dst = torch.full((rec.size,), -99, dtype=torch.int32, device="cuda")
    out = []
    for src, record in ((drec, None), (host, (host, dst))):
        kc, vc = (torch.zeros((40, Hkv, D), device="cuda") for _ in range(2))
        q = torch.empty((rows, H * D), device="cuda")
        x = torch.full((rows, k), float("nan"), device="cuda")
        o.qkv_rope_cache(q, kc, vc, table, w, g, src[rows:2 * rows], src[2 * rows:3 * rows],
                         cos, sin, H, Hkv, D, row_index=src[:rows], x_out=x, prev_ids=prev,
                         record=record)
        out.append((q, kc, vc, x))
    torch.cuda.synchronize()
    for a, b in zip(*out):
        assert torch.equal(a, b)
    assert torch.equal(dst.cpu(), torch.from_numpy(rec))

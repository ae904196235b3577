"""vl_paged_attention_noalloc, the allocation-free entry point, through the C
ABI: its output equals vl_paged_attention's with a caller workspace of the
same size, bit for bit, and meets the oracle's bf16 / fp32 row bars, on two
calls in a row with the second batch smaller than the first (the static
scratch keeps the first call's contents). Batches whose plan cannot fit the
scratch are rejected before anything is launched."""

import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from batches import bf16_round, make_batch, oracle_attention  # noqa: E402
from parity import BF16_ROW_REL, F32_ROW_REL, assert_rows_close  # noqa: E402

pytestmark = pytest.mark.gpu


def _run_both(b, dtype):
    from vllmlite_amd import ops
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    q = torch.from_numpy(b["q"]).cuda().to(tdt)
    kc = torch.from_numpy(b["k_cache"]).cuda().to(tdt)
    vc = torch.from_numpy(b["v_cache"]).cuda().to(tdt)
    bt = torch.from_numpy(b["block_tables"]).cuda()
    sl = torch.from_numpy(b["seq_lens"]).cuda()
    qsl = torch.from_numpy(b["qsl"]).cuda()
    q_lens = np.diff(b["qsl"])
    max_q, min_q = int(q_lens.max()), int(q_lens[q_lens > 0].min())
    got = torch.full_like(q, float("nan"))
    ops.paged_attention_noalloc(got, q, kc, vc, bt, sl, qsl, b["scale"], b["bs"], max_q, min_q)
    ws = torch.empty(ops.NOALLOC_SCRATCH_BYTES, dtype=torch.uint8, device="cuda")
    ref = torch.full_like(q, float("nan"))
    ops.paged_attention(ref, q, kc, vc, bt, sl, qsl, b["scale"], b["bs"], ws, max_q, min_q)
    torch.cuda.synchronize()
    return got.float().cpu().numpy(), ref.float().cpu().numpy()


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_noalloc_matches_workspace_call_twice(dtype):
    first = [(1, 5000), (5, 3000), (1, 70), (64, 700), (1, 8192), (17, 17)] + [(1, 300)] * 40
    second = [(1, 900), (3, 40), (1, 16)]
    for seqs, seed in ((first, 80), (second, 81)):
        b = make_batch(seqs, 32, 8, 128, 16, seed=seed)
        got, ref = _run_both(b, dtype)
        assert np.array_equal(got, ref, equal_nan=False), "differs from vl_paged_attention"
        if dtype == "f32":
            assert_rows_close(got, oracle_attention(b), F32_ROW_REL)
        else:
            want = oracle_attention(b, bf16_round(b["q"]), bf16_round(b["k_cache"]),
                                    bf16_round(b["v_cache"]))
            assert_rows_close(got, want, BF16_ROW_REL)


def test_noalloc_rejects_batches_beyond_its_scratch():
    from vllmlite_amd import ops
    lib = ops.lib()
    n = 2_000_000  # its plan alone needs ~112 MB, beyond the 32 MiB scratch
    assert lib.vl_paged_attention_min_workspace(n) > ops.NOALLOC_SCRATCH_BYTES
    rc = lib.vl_paged_attention_noalloc(None, None, 0, None, None, None, 0, None, None, n, n,
                                        32, 8, 128, 16, 1.0, 1, 0, 1, 1, 0, None)
    assert rc == -1 and b"static scratch" in lib.vl_last_error()

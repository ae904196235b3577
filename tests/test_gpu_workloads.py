"""The benchmark workloads at full size on the GPU, checked against the oracle.

Each builds the batch in a 2^17-block pool (8.6 GB of bf16 K/V, unowned slots
NaN), runs the step through the C ABI and compares EVERY sequence with the
oracle's per-sequence paged_attention (vllmlite/attention.py:59-98) on fp32
copies of the same bf16 values, each (token, head) row within 2e-2 normwise
(tests/parity.py). The K/V scatter is checked bit-exact.
"""

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from parity import BF16_ROW_REL, assert_rows_close  # noqa: E402

pytestmark = pytest.mark.gpu


def _mods():
    from vllmlite_amd import ops
    from vllmlite_amd import synthetic as syn
    return ops, syn


def _oracle_rows(b, i):
    from oracle.attention import gather_slots, paged_attention
    nb = (int(b["ctx"][i]) + b["bs"] - 1) // b["bs"]
    slots = gather_slots(b["tables_np"][i, :nb], b["bs"], int(b["ctx"][i]))
    sl = torch.from_numpy(slots).cuda()
    k = b["kc"][sl].float().cpu().numpy()
    v = b["vc"][sl].float().cpu().numpy()
    q0, q1 = b["qsl_np"][i], b["qsl_np"][i + 1]
    q = b["q"][q0:q1].float().cpu().numpy()
    return paged_attention(q, k, v, np.arange(len(slots)), b["Hkv"], b["scale"])


def _step(ops, syn, b, scatter=True):
    S, T = len(b["seqs"]), int(b["q_lens"].sum())
    ws = ops.AttentionWorkspace().get(
        ops.paged_attention_workspace_size(S, T, b["H"], b["D"], int(b["ctx"].max())))
    out = torch.empty_like(b["q"])
    if scatter:
        ops.reshape_and_cache(b["knew"], b["vnew"], b["kc"], b["vc"], b["slot_mapping"])
    ops.paged_attention(out, b["q"], b["kc"], b["vc"], b["bt"], b["seq_lens"], b["qsl"],
                        b["scale"], b["bs"], ws, max_query_len=b["max_q"],
                        min_query_len=b["min_q"])
    torch.cuda.synchronize()
    return out


def _check(b, out, idx=None):
    """Sequences idx (default: all) against the oracle; returns the worst row error."""
    worst = 0.0
    for i in (range(len(b["seqs"])) if idx is None else idx):
        q0, q1 = b["qsl_np"][i], b["qsl_np"][i + 1]
        got = out[q0:q1].float().cpu().numpy()
        worst = max(worst, assert_rows_close(
            got, _oracle_rows(b, i), BF16_ROW_REL,
            f"sequence {i} (q={b['q_lens'][i]}, ctx={b['ctx'][i]})"))
    return worst


def test_mixed_8392_step_scatter_and_attention():
    """16 chunks x 512 tokens after 0-2048 cached tokens plus 200 decodes with
    128-4096 tokens, one scatter and one attention call: every sequence
    against the oracle, the scatter bit-exact."""
    ops, syn = _mods()
    b = syn.build(torch, syn.mixed_8392_seqs(0), seed=2)
    out = _step(ops, syn, b)
    sm = b["slot_mapping"].long()
    assert torch.equal(b["kc"][sm], b["knew"]) and torch.equal(b["vc"][sm], b["vnew"])
    print("worst row error", _check(b, out))
    del b, out
    torch.cuda.empty_cache()


def test_verify_64x5_step():
    """64 sequences x 5 query positions over 1024-32768 cached tokens: every
    sequence against the oracle."""
    ops, syn = _mods()
    b = syn.build(torch, syn.verify_64x5_seqs(0), seed=3)
    out = _step(ops, syn, b)
    print("worst row error", _check(b, out))
    del b, out
    torch.cuda.empty_cache()


def test_decode_256_step():
    """The headline decode batch: all 256 sequences against the oracle."""
    ops, syn = _mods()
    b = syn.build(torch, syn.decode_256_seqs(0), seed=0)
    out = _step(ops, syn, b)
    print("worst row error", _check(b, out))
    del b, out
    torch.cuda.empty_cache()

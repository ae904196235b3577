"""The one-launch decode step (vl_decode_step: the whole TinyLlama forward of
a step whose sequences each push one token, vllmlite/model.py:80-120, plus
the argmax of every row, vllmlite/sampling.py:56-57) against the same steps
on this library's separate kernels, and end to end against the reference.

Both runners see the same scheduled batches (the engine drives the first and
the second is handed each batch too), and before each step the second's
caches are set to the first's, so every comparison is of one step from the
same cache (a narrow cache's rounding, once it differs, would otherwise carry
into every later step).
The projections are the same operations in the same order; the attention
sums in another order, so every decode step's logits must agree within 1e-5
of the row's largest logit (1e-3 with a bf16 or FP8 cache), and the ids equal the host argmax of the
separate kernels' logits wherever that row's top-1 / top-2 margin exceeds
1e-4 (a near-tie may go either way)."""

import json
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from vllmlite_amd.engine import LLMEngine  # noqa: E402
from vllmlite_amd.request import SamplingParams  # noqa: E402
from vllmlite_amd.workload import mixed_lengths  # noqa: E402

from helpers import PROMPTS, cfg0_config, small_cfg  # noqa: E402

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


class _Twin:
    """execute() / execute_argmax() on the one-launch runner, each batch also
    run through a runner without it; every result compared."""

    def __init__(self, cfg, tol=1e-5):
        from vllmlite_amd.hip_runner import HipRunner
        self.tol = tol
        self.a = HipRunner(cfg.model, cfg.cache, one_launch_decode=True)
        self.b = HipRunner(cfg.model, cfg.cache, one_launch_decode=False)
        assert self.a._step is not None, "no one-launch kernel for this shape"
        self.vocab_size = self.a.vocab_size
        self.decode_steps = 0

    def _same_caches(self):
        torch.cuda.synchronize()
        self.b.cache_k.copy_(self.a.cache_k)
        self.b.cache_v.copy_(self.a.cache_v)
        torch.cuda.synchronize()

    def execute(self, out):
        n0 = self.a.one_launch_steps
        self._same_caches()
        la, rows = self.a.execute(out)
        lb, rows_b = self.b.execute(out)
        assert rows == rows_b
        if self.a.one_launch_steps > n0:
            self.decode_steps += 1
            scale = np.abs(lb).max(axis=-1, keepdims=True)
            assert np.all(np.abs(la - lb) <= self.tol * scale), np.abs(la - lb).max()
        return la, rows

    def execute_argmax(self, out):
        n0 = self.a.one_launch_steps
        self._same_caches()
        ia, rows = self.a.execute_argmax(out)
        lb, _ = self.b.execute(out)
        if self.a.one_launch_steps > n0:
            self.decode_steps += 1
        want = np.argmax(lb, axis=-1)
        top2 = np.sort(lb, axis=-1)[:, -2:]
        clear = top2[:, 1] - top2[:, 0] > 1e-4
        assert np.array_equal(ia[clear], want[clear])
        return ia, rows


def _drive(cfg, reqs, argmax, tol=1e-5):
    twin = _Twin(cfg, tol)
    eng = LLMEngine(cfg, runner=twin, lookahead=False)
    eng.device_argmax = argmax
    for rid, ids, p in reqs:
        eng.add_request(params=p, request_id=rid, prompt_token_ids=ids)
    while eng.has_work:
        eng.step()
    return eng, twin


@pytest.mark.parametrize("layout", ["token", "head"])
def test_cfg0_mix_decode_steps_equal_separate_kernels(layout):
    """The 48-request TinyLlama mix (6 layers, d 384, H8/Hkv4, d_ff 1024):
    228 decode steps in one launch each, logits those of the separate
    kernels, streams the reference's."""
    g = json.load(open(os.path.join(GOLD, "cfg0_streams.json")))
    cfg = cfg0_config(False)
    cfg.cache.kv_layout = layout
    eng, twin = _drive(cfg, mixed_lengths(0, 48, 0), argmax=False)
    assert twin.decode_steps >= 200, twin.decode_steps
    for rid, want in g["streams"].items():
        assert eng.seqs[rid].output_token_ids == want, rid


def test_cfg0_mix_device_argmax_ids():
    """The same mix through execute_argmax: the one-launch kernel's ids are the
    argmax of the separate kernels' logits, row for row."""
    _, twin = _drive(cfg0_config(False), mixed_lengths(0, 48, 0)[:20], argmax=True)
    assert twin.decode_steps >= 100


@pytest.mark.parametrize("kv_dtype", ["bfloat16", "float8_e4m3"])
def test_narrow_cache_decode_steps_equal_separate_kernels(kv_dtype):
    """bf16 and FP8 E4M3 caches: the one-launch kernel rounds the K/V it
    writes as the separate kernels do, and widens the cache the same way.
    Bar 1e-3 of the row's largest logit, as for the narrow caches against the
    oracle runner: K/V computed from inputs ~1e-6 apart can round one cache
    step apart."""
    cfg = cfg0_config(False)
    cfg.cache.kv_dtype = kv_dtype
    _, twin = _drive(cfg, mixed_lengths(0, 48, 0)[:24], argmax=False, tol=1e-3)
    assert twin.decode_steps >= 100


@pytest.mark.parametrize("block_size", [1, 4, 16, 64])
def test_small_model_decode_steps_equal_separate_kernels(block_size):
    """head_dim 16 (2 layers, d 64, H4/Hkv2), block sizes 1..64."""
    cfg = small_cfg(block_size=block_size)
    p = SamplingParams(max_tokens=20, temperature=0.0, ignore_eos=True)
    reqs = [(f"r{i}", [1] + [ord(c) for c in x], p) for i, x in enumerate(PROMPTS)]
    _, twin = _drive(cfg, reqs, argmax=False)
    assert twin.decode_steps >= 15


def test_one_launch_steps_in_the_lookahead_engine():
    """With lookahead (the default engine), decode steps go through
    launch_argmax / collect as one launch each; streams are the reference's."""
    from vllmlite_amd.hip_runner import HipRunner
    g = json.load(open(os.path.join(GOLD, "cfg0_streams.json")))
    cfg = cfg0_config(False)
    runner = HipRunner(cfg.model, cfg.cache, one_launch_decode=True)
    eng = LLMEngine(cfg, runner=runner)
    for rid, ids, p in mixed_lengths(0, 48, 0):
        eng.add_request(params=p, request_id=rid, prompt_token_ids=ids)
    while eng.has_work:
        eng.step()
    assert runner.one_launch_steps >= 200
    for rid, want in g["streams"].items():
        assert eng.seqs[rid].output_token_ids == want, rid

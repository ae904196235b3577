"""The oracle's bf16 rounding (the values a bf16 K/V cache holds) against
torch's bfloat16 conversion and hand-picked ties, and the oracle runner with a
bf16 cache: its cache holds only bf16 values and its greedy streams stay close
to the fp32 runner's."""

import numpy as np
import pytest

from oracle.attention import round_bf16

torch = pytest.importorskip("torch")


def test_round_bf16_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32),
        (rng.standard_normal(1000) * 1e30).astype(np.float32),
        (rng.standard_normal(1000) * 1e-38).astype(np.float32),  # subnormals
        np.array([0.0, -0.0, np.inf, -np.inf, 3.3895314e38, -3.3895314e38], np.float32),
    ])
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = round_bf16(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_round_bf16_ties_go_to_even():
    one = np.float32(1.0)
    ulp = np.float32(2.0 ** -7)  # bf16 spacing at 1.0
    x = np.array([one + ulp / 2, one + 3 * ulp / 2, one + ulp / 2 + 2.0 ** -20, -(one + ulp / 2)],
                 np.float32)
    assert round_bf16(x).tolist() == [1.0, 1.0 + 2 * ulp, 1.0 + ulp, -1.0]
    assert np.isnan(round_bf16(np.array([np.nan], np.float32)))[0]


def test_numpy_runner_bf16_cache_holds_bf16_values():
    from helpers import PROMPTS, run, small_cfg
    from oracle.runner import NumpyRunner
    from vllmlite_amd.engine import LLMEngine
    cfg = small_cfg()
    cfg.cache.kv_dtype = "bfloat16"
    eng = LLMEngine(cfg, runner=NumpyRunner(cfg.model, cfg.cache))
    out = run(eng, PROMPTS, max_tokens=8)
    ck = eng.runner.cache_k
    assert np.any(ck != 0) and np.array_equal(round_bf16(ck), ck)
    fp32 = run(LLMEngine(small_cfg(), runner=NumpyRunner(small_cfg().model, small_cfg().cache)),
               PROMPTS, max_tokens=8)
    assert sum(a == b for a, b in zip(out, fp32)) >= len(PROMPTS) - 1

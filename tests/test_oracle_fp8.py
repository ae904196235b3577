"""The oracle's FP8 E4M3 rounding (the values an FP8 K/V cache holds) pinned
by the format's closed forms, round trips of every code, ties, saturation and
torch's float8_e4m3fn conversion; and the oracle runner with an FP8 cache."""

import numpy as np
import pytest

from oracle.attention import fp8_e4m3_decode, fp8_e4m3_encode, round_fp8_e4m3

torch = pytest.importorskip("torch")


def test_decode_closed_forms():
    v = fp8_e4m3_decode(np.array([0x00, 0x01, 0x07, 0x08, 0x0F, 0x38, 0x3C, 0x77, 0x7E, 0x80,
                                  0xB8, 0xFE], np.uint8))
    want = [0.0, 2.0 ** -9, 7 * 2.0 ** -9, 2.0 ** -6, 1.875 * 2.0 ** -6, 1.0, 1.5, 1.875 * 128,
            448.0, -0.0, -1.0, -448.0]
    assert v.tolist() == want
    assert np.signbit(v[9])
    assert np.isnan(fp8_e4m3_decode(np.array([0x7F, 0xFF], np.uint8))).all()
    pos = fp8_e4m3_decode(np.arange(0x7F, dtype=np.uint8))
    assert np.all(np.diff(pos) > 0)  # codes 0x00..0x7E increase strictly


def test_every_finite_code_round_trips():
    codes = np.arange(256, dtype=np.uint8)
    fin = (codes & 0x7F) != 0x7F
    assert np.array_equal(fp8_e4m3_encode(fp8_e4m3_decode(codes[fin])), codes[fin])


def test_ties_go_to_the_even_code_and_others_to_the_nearest():
    pos = fp8_e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mid = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)  # every midpoint is an fp32 value
    assert np.array_equal(mid.astype(np.float64), (pos[:-1] + pos[1:]) / 2)
    lower = np.arange(0x7E)
    even = np.where(lower % 2 == 0, lower, lower + 1)
    assert np.array_equal(fp8_e4m3_encode(mid), even)
    assert np.array_equal(fp8_e4m3_encode(-mid), even | 0x80)
    up = np.nextafter(mid, np.float32(np.inf))
    down = np.nextafter(mid, np.float32(0))
    assert np.array_equal(fp8_e4m3_encode(up), lower + 1)
    assert np.array_equal(fp8_e4m3_encode(down), lower)


def test_saturation_and_nan():
    x = np.array([448.0, 460.0, 464.0, 470.0, 1e6, np.inf, -np.inf, -1e30, np.nan, -np.nan],
                 np.float32)
    got = fp8_e4m3_encode(x)
    assert got[:6].tolist() == [0x7E] * 6 and got[6:8].tolist() == [0xFE] * 2
    assert (got[8:] & 0x7F).tolist() == [0x7F, 0x7F]


def test_matches_torch_float8_e4m3fn_in_range():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * s
                        for s in (1e-3, 0.05, 1.0, 60.0)])
    x = x[np.abs(x) < 448]
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(fp8_e4m3_encode(x), want)
    assert np.array_equal(round_fp8_e4m3(x).view(np.uint32),
                          torch.from_numpy(x).to(torch.float8_e4m3fn).float().numpy().view(np.uint32))


def test_numpy_runner_fp8_cache_holds_fp8_values():
    from helpers import PROMPTS, run, small_cfg
    from oracle.runner import NumpyRunner
    from vllmlite_amd.engine import LLMEngine
    cfg = small_cfg()
    cfg.cache.kv_dtype = "float8_e4m3"
    eng = LLMEngine(cfg, runner=NumpyRunner(cfg.model, cfg.cache))
    out = run(eng, PROMPTS, max_tokens=8)
    ck = eng.runner.cache_k
    assert np.any(ck != 0) and np.array_equal(round_fp8_e4m3(ck), ck)
    assert all(len(o) == 8 for o in out)

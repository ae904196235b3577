"""Closed forms that pin the oracle's RMSNorm and SiLU (vllmlite/model.py:17-23)."""

import numpy as np

from oracle.model import rms_norm, silu


def test_rms_norm_known_answer():
    # mean of squares of (3, 4) is 12.5: each element divided by sqrt(12.5 + 1e-5)
    x = np.array([[3.0, 4.0]], np.float32)
    w = np.array([1.0, 2.0], np.float32)
    want = np.array([[3.0, 8.0]]) / np.sqrt(12.5 + 1e-5)
    np.testing.assert_allclose(rms_norm(x, w), want, rtol=1e-6)


def test_rms_norm_unit_rms_and_scale_invariance():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((7, 384)) * 5).astype(np.float32)
    y = rms_norm(x, np.ones(384, np.float32))
    np.testing.assert_allclose(np.sqrt((y.astype(np.float64) ** 2).mean(axis=-1)), 1.0, rtol=1e-5)
    np.testing.assert_allclose(rms_norm(3 * x, np.ones(384, np.float32)), y, rtol=1e-5, atol=1e-6)
    # the normalisation is per row: rows do not mix
    np.testing.assert_allclose(rms_norm(x[2:3], np.ones(384, np.float32)), y[2:3], rtol=1e-6)


def test_rms_norm_eps_matters_near_zero():
    x = np.full((1, 4), 1e-4, np.float32)
    # mean square 1e-8 against eps 1e-5: the output is x / sqrt(1.001e-5), far from 1
    np.testing.assert_allclose(rms_norm(x, np.ones(4, np.float32)), x / np.sqrt(1e-8 + 1e-5),
                               rtol=1e-5)


def test_silu_closed_forms():
    x = np.linspace(-20, 20, 401).astype(np.float32)
    s = silu(x).astype(np.float64)
    assert silu(np.zeros(1, np.float32))[0] == 0.0
    # silu(x) - silu(-x) = x (sigma(x) + sigma(-x) = 1)
    np.testing.assert_allclose(s - silu(-x).astype(np.float64), x, atol=2e-5)
    # silu(1) = 1 / (1 + e^-1)
    np.testing.assert_allclose(silu(np.ones(1, np.float32)), 1 / (1 + np.exp(-1.0)), rtol=1e-6)
    assert (s[x > 0] > 0).all() and abs(s.min() - (-0.2784645)) < 1e-4  # minimum near x = -1.278

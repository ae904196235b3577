"""Parity bars for attention outputs.

Attention outputs are averages over the context, so their magnitude shrinks
like sqrt(1/ctx): at 32K keys a typical element is ~0.007. An elementwise
absolute tolerance cannot see a kernel that loses part of the context at that
scale. Every (token, head) row is therefore checked on its own, normwise:

    ||got_row - want_row||_2 <= rel * ||want_row||_2

with rel = 2e-2 for bf16 (the kernels read bf16 K/V, round probabilities to
bf16 for the PV product and store bf16) and 1e-4 for fp32, the two bars the
paged-attention path is held to.
"""

from __future__ import annotations

import numpy as np

BF16_ROW_REL = 2e-2
F32_ROW_REL = 1e-4


def row_rel_err(got: np.ndarray, want: np.ndarray) -> np.ndarray:
    """Normwise relative error of every row along the last axis."""
    g = np.asarray(got, dtype=np.float64).reshape(-1, got.shape[-1])
    w = np.asarray(want, dtype=np.float64).reshape(-1, want.shape[-1])
    num = np.linalg.norm(g - w, axis=1)
    den = np.linalg.norm(w, axis=1)
    return num / np.maximum(den, 1e-30)


def assert_rows_close(got: np.ndarray, want: np.ndarray, rel: float, what: str = "") -> float:
    """Fails unless every row of got [.., H, D] is finite and within `rel` of
    the same row of want, normwise. Returns the worst row error."""
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = row_rel_err(got, want)
    worst = int(np.argmax(err)) if err.size else 0
    if err.size:
        heads = got.shape[-2] if got.ndim >= 2 else 1
        assert err[worst] <= rel, (
            f"{what}: token {worst // heads} head {worst % heads}: normwise error "
            f"{err[worst]:.3g} > {rel}")
        return float(err[worst])
    return 0.0

"""Weights from an .npz (vllmlite/model.py:60-71, runner.py:41-44): what
init_weights draws survives a save / load round trip bit for bit, a file
without lm_head ties it to tok_emb^T, other float widths are read as fp32,
and object arrays are refused (numpy's allow_pickle=False)."""

import dataclasses
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "vllm-lite_amd"))

from vllmlite_amd.config import ModelConfig  # noqa: E402
from vllmlite_amd.model import LAYER_KEYS, init_weights, load_weights, model_weights  # noqa: E402


def _cfg(**kw):
    return ModelConfig(n_layers=2, n_heads=4, n_kv_heads=2, d_model=64, d_ff=128,
                       max_seq_len=512, **kw)


def test_npz_round_trip_is_exact(tmp_path):
    cfg = _cfg()
    w = init_weights(cfg)
    path = tmp_path / "w.npz"
    np.savez(path, **w)
    got = load_weights(cfg, str(path))
    assert sorted(got) == sorted(w)
    for k in w:
        assert got[k].dtype == np.float32 and np.array_equal(got[k], w[k]), k


def test_weights_path_selects_the_file(tmp_path):
    cfg = _cfg()
    other = init_weights(dataclasses.replace(cfg, seed=7))
    path = tmp_path / "other.npz"
    np.savez(path, **other)
    got = model_weights(dataclasses.replace(cfg, weights_path=str(path)))
    assert all(np.array_equal(got[k], other[k]) for k in other)
    assert not np.array_equal(model_weights(cfg)["tok_emb"], other["tok_emb"])


def test_missing_lm_head_is_tied_and_widths_are_cast(tmp_path):
    cfg = _cfg()
    w = init_weights(cfg)
    stored = {k: v.astype(np.float64) for k, v in w.items() if k != "lm_head"}
    path = tmp_path / "tied.npz"
    np.savez(path, **stored)
    got = load_weights(cfg, str(path))
    assert got["lm_head"].dtype == np.float32
    assert np.array_equal(got["lm_head"], w["tok_emb"].T)
    for i in range(cfg.n_layers):
        for k in LAYER_KEYS:
            assert np.array_equal(got[f"layers.{i}.{k}"], w[f"layers.{i}.{k}"])


def test_object_arrays_are_refused(tmp_path):
    cfg = _cfg()
    w = init_weights(cfg)
    w["tok_emb"] = np.array([object()] * 3, dtype=object)
    path = tmp_path / "pickled.npz"
    np.savez(path, **w)
    with pytest.raises(ValueError):
        load_weights(cfg, str(path))


def test_missing_layer_raises(tmp_path):
    cfg = _cfg()
    w = init_weights(cfg)
    del w["layers.1.w_down"]
    path = tmp_path / "short.npz"
    np.savez(path, **w)
    with pytest.raises(KeyError):
        load_weights(cfg, str(path))

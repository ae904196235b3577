"""TinyLlama weights and tables for the device forward.

The decoder is the reference's (vllmlite/model.py:26-120): RMSNorm (eps 1e-5),
interleaved RoPE, GQA attention, SwiGLU MLP, tied lm_head. This module owns
the host side of it:

  init_weights   seeded random weights, drawn from default_rng(cfg.seed) in
                 the reference's order (model.py:50-55, 32-43) so that a
                 given ModelConfig yields the same numbers: tok_emb [V, d]
                 with std d^-1/2; per layer wq, wk, wv, wo, w_gate, w_up with
                 std d^-1/2 and w_down [d_ff, d] with std d_ff^-1/2; norm
                 weights ones; lm_head = tok_emb^T.
  load_weights   the same dictionary from an .npz (model.py:64-71), read with
                 numpy's default allow_pickle=False.
  rope_tables    fp32 cos/sin [max_pos, head_dim/2] with angles pos * theta^(-2i/D)
                 computed in float32 (attention.py:21-25); uploaded once, so
                 the device rotates with the host's exact table values.
  pack_weights   fused [d, (H+2Hkv)*hd] QKV and [d, 2*d_ff] gate|up matrices,
                 fp32, on the device.
"""

from __future__ import annotations

from typing import Dict

import numpy as np

LAYER_KEYS = ("attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "w_gate", "w_up", "w_down")


def init_weights(cfg) -> Dict[str, np.ndarray]:
    rng = np.random.default_rng(cfg.seed)
    d, hd, f = cfg.d_model, cfg.head_dim, cfg.d_ff
    std = 1.0 / np.sqrt(d)

    def normal(*shape):
        return (rng.standard_normal(shape) * std).astype(np.float32)

    w = {"tok_emb": normal(cfg.vocab_size, d)}
    for i in range(cfg.n_layers):
        p = f"layers.{i}."
        w[p + "attn_norm"] = np.ones(d, np.float32)
        w[p + "wq"] = normal(d, cfg.n_heads * hd)
        w[p + "wk"] = normal(d, cfg.n_kv_heads * hd)
        w[p + "wv"] = normal(d, cfg.n_kv_heads * hd)
        w[p + "wo"] = normal(cfg.n_heads * hd, d)
        w[p + "ffn_norm"] = np.ones(d, np.float32)
        w[p + "w_gate"] = normal(d, f)
        w[p + "w_up"] = normal(d, f)
        w[p + "w_down"] = (rng.standard_normal((f, d)) / np.sqrt(f)).astype(np.float32)
    w["final_norm"] = np.ones(d, np.float32)
    w["lm_head"] = np.ascontiguousarray(w["tok_emb"].T)
    return w


def load_weights(cfg, path: str) -> Dict[str, np.ndarray]:
    z = np.load(path)
    w = {"tok_emb": z["tok_emb"].astype(np.float32),
         "final_norm": z["final_norm"].astype(np.float32)}
    w["lm_head"] = (z["lm_head"].astype(np.float32) if "lm_head" in z.files
                    else np.ascontiguousarray(w["tok_emb"].T))
    for i in range(cfg.n_layers):
        for k in LAYER_KEYS:
            w[f"layers.{i}.{k}"] = z[f"layers.{i}.{k}"].astype(np.float32)
    return w


def model_weights(cfg) -> Dict[str, np.ndarray]:
    """Random seeded weights, or cfg.weights_path when set (model.py:60-61)."""
    return load_weights(cfg, cfg.weights_path) if cfg.weights_path else init_weights(cfg)


def rope_tables(head_dim: int, max_pos: int, theta: float = 10000.0):
    exponent = np.arange(0, head_dim, 2, dtype=np.float32) / head_dim
    inv_freq = 1.0 / (theta ** exponent)
    angles = np.arange(max_pos, dtype=np.float32)[:, None] * inv_freq[None, :]
    return np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)


def pack_weights(cfg, w: Dict[str, np.ndarray], torch, device) -> dict:
    """Device copies: per layer fused qkv / gate_up matrices plus the rest."""

    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)

    layers = []
    for i in range(cfg.n_layers):
        p = f"layers.{i}."
        layers.append({
            "attn_norm": dev(w[p + "attn_norm"]),
            "w_qkv": dev(np.concatenate([w[p + "wq"], w[p + "wk"], w[p + "wv"]], axis=1)),
            "wo": dev(w[p + "wo"]),
            "ffn_norm": dev(w[p + "ffn_norm"]),
            "w_gate_up": dev(np.concatenate([w[p + "w_gate"], w[p + "w_up"]], axis=1)),
            "w_down": dev(w[p + "w_down"]),
        })
    return {"tok_emb": dev(w["tok_emb"]), "lm_head": dev(w["lm_head"]),
            "final_norm": dev(w["final_norm"]), "layers": layers}


def tile_weights(packed: dict, tile16, torch) -> None:
    """Add 16-column tiled copies of the projection weights (suffix `_t`) for
    the decode-step kernels, which read them in whole cache lines. Each kind
    (the norm weights and the tiled projections) is then stacked into one
    [n_layers, ...] buffer (packed["stacked"]), and the per-layer entries
    become views of it: the one-launch decode step finds a layer's weights at
    a fixed stride from the first."""
    layers = packed["layers"]
    for L in layers:
        L["w_qkv_t"] = tile16(L["w_qkv"])
        L["wo_t"] = tile16(L["wo"])
        L["w_gate_up_t"] = tile16(L["w_gate_up"], 2)
        L["w_down_t"] = tile16(L["w_down"])
    packed["lm_head_t"] = tile16(packed["lm_head"])
    packed["stacked"] = {}
    for key in ("attn_norm", "w_qkv_t", "wo_t", "ffn_norm", "w_gate_up_t", "w_down_t"):
        all_ = torch.stack([L[key] for L in layers]).contiguous()
        packed["stacked"][key] = all_
        for i, L in enumerate(layers):
            L[key] = all_[i]

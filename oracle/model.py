"""NumPy restatement of the TinyLlama decoder (vllmlite/model.py:17-120).
Test infrastructure only.

Weights are drawn from default_rng(seed) in the reference's order
(model.py:50-55, 32-43): tok_emb [V, d] * d^-1/2; then per layer wq, wk, wv,
wo, w_gate, w_up with std d^-1/2 and w_down with std d_ff^-1/2; norms are
ones; lm_head is tok_emb.T (tied). Matrices are stored [in, out].
"""

from __future__ import annotations

import numpy as np

from .attention import apply_rope, build_rope, paged_attention, write_kv

LAYER_KEYS = ("attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "w_gate", "w_up", "w_down")


def rms_norm(x, w, eps: float = 1e-5):
    """model.py:17-19."""
    var = np.mean(x * x, axis=-1, keepdims=True)
    return (x / np.sqrt(var + eps)) * w


def silu(x):
    """model.py:22-23."""
    return x / (1.0 + np.exp(-x))


def init_weights(cfg) -> dict:
    rng = np.random.default_rng(cfg.seed)
    d, hd, f = cfg.d_model, cfg.head_dim, cfg.d_ff
    s = 1.0 / np.sqrt(d)
    w = {"tok_emb": (rng.standard_normal((cfg.vocab_size, d)) * s).astype(np.float32)}
    for i in range(cfg.n_layers):
        g = lambda *shape: (rng.standard_normal(shape) * s).astype(np.float32)
        w[f"layers.{i}.attn_norm"] = np.ones(d, dtype=np.float32)
        w[f"layers.{i}.wq"] = g(d, cfg.n_heads * hd)
        w[f"layers.{i}.wk"] = g(d, cfg.n_kv_heads * hd)
        w[f"layers.{i}.wv"] = g(d, cfg.n_kv_heads * hd)
        w[f"layers.{i}.wo"] = g(cfg.n_heads * hd, d)
        w[f"layers.{i}.ffn_norm"] = np.ones(d, dtype=np.float32)
        w[f"layers.{i}.w_gate"] = g(d, f)
        w[f"layers.{i}.w_up"] = g(d, f)
        w[f"layers.{i}.w_down"] = (rng.standard_normal((f, d)) / np.sqrt(f)).astype(np.float32)
    w["final_norm"] = np.ones(d, dtype=np.float32)
    w["lm_head"] = w["tok_emb"].T.copy()
    return w


class TinyLlamaOracle:
    def __init__(self, cfg, weights: dict | None = None, kv_round=None):
        self.cfg = cfg
        self.w = weights if weights is not None else init_weights(cfg)
        # applied to K/V rows as they are cached (round_bf16 for a bf16 cache)
        self.kv_round = kv_round if kv_round is not None else (lambda a: a)
        self.cos, self.sin = build_rope(cfg.head_dim, cfg.max_seq_len)
        self.scale = 1.0 / np.sqrt(cfg.head_dim)
        self.layers = [{k: self.w[f"layers.{i}.{k}"] for k in LAYER_KEYS}
                       for i in range(cfg.n_layers)]

    def forward(self, token_ids, positions, cache_k, cache_v, seq_meta, last_idx):
        """model.py:80-120. seq_meta: (start, q_len, write_slots, read_slots) per sequence."""
        cfg = self.cfg
        hd = cfg.head_dim
        x = self.w["tok_emb"][token_ids]
        for li, L in enumerate(self.layers):
            h = rms_norm(x, L["attn_norm"])
            q = (h @ L["wq"]).reshape(-1, cfg.n_heads, hd)
            k = (h @ L["wk"]).reshape(-1, cfg.n_kv_heads, hd)
            v = (h @ L["wv"]).reshape(-1, cfg.n_kv_heads, hd)
            q = apply_rope(q, positions, self.cos, self.sin)
            k = apply_rope(k, positions, self.cos, self.sin)
            ck, cv = cache_k[li], cache_v[li]
            attn = np.empty_like(q)
            for start, q_len, wslots, rslots in seq_meta:
                sl = slice(start, start + q_len)
                write_kv(ck, cv, self.kv_round(k[sl]), self.kv_round(v[sl]), wslots)
                attn[sl] = paged_attention(q[sl], ck, cv, rslots, cfg.n_kv_heads, self.scale)
            x = x + attn.reshape(-1, cfg.n_heads * hd) @ L["wo"]
            h = rms_norm(x, L["ffn_norm"])
            x = x + (silu(h @ L["w_gate"]) * (h @ L["w_up"])) @ L["w_down"]
        tail = rms_norm(x[last_idx], self.w["final_norm"])
        return tail @ self.w["lm_head"]

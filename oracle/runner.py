"""NumPy model runner (vllmlite/runner.py:35-100). Test infrastructure only:
the CPU oracle for HipRunner and the timed CPU baseline in bench.py."""

from __future__ import annotations

import numpy as np

from .attention import gather_slots, round_bf16, round_fp8_e4m3
from .model import TinyLlamaOracle


class NumpyRunner:
    """Same interface as the package's ModelRunner: execute(out) -> (logits, rows)."""

    def __init__(self, model_cfg, cache_cfg, weights: dict | None = None):
        self.model_cfg = model_cfg
        self.block_size = cache_cfg.block_size
        # a bf16 or FP8 E4M3 K/V cache (cache_cfg.kv_dtype "bfloat16",
        # "float8_e4m3"): the fp32 cache arrays hold K/V rounded to it when written
        kv_round = {"bfloat16": round_bf16, "float8_e4m3": round_fp8_e4m3}.get(
            getattr(cache_cfg, "kv_dtype", "float32"))
        self.model = TinyLlamaOracle(model_cfg, weights, kv_round)
        shape = (model_cfg.n_layers, cache_cfg.num_blocks * cache_cfg.block_size,
                 model_cfg.n_kv_heads, model_cfg.head_dim)
        self.cache_k = np.zeros(shape, dtype=np.float32)
        self.cache_v = np.zeros(shape, dtype=np.float32)
        self.last_batch = None  # (token_ids, positions, seq_meta, want) of the last step

    @property
    def vocab_size(self) -> int:
        return self.model_cfg.vocab_size

    @property
    def cache_bytes(self) -> int:
        return self.cache_k.nbytes + self.cache_v.nbytes

    def do_cow(self, pairs) -> None:
        """runner.py:54-60: in list order, copy one block's slots across all layers."""
        bs = self.block_size
        for src, dst in pairs:
            s = slice(src * bs, (src + 1) * bs)
            d = slice(dst * bs, (dst + 1) * bs)
            self.cache_k[:, d] = self.cache_k[:, s]
            self.cache_v[:, d] = self.cache_v[:, s]

    def execute(self, out):
        if out.cow:
            self.do_cow(out.cow)
        token_ids, positions, seq_meta, want, rows = [], [], [], [], []
        for item in out.scheduled:
            seq = item.seq
            start = seq.num_computed
            n = item.num_tokens
            offset = len(token_ids)
            token_ids += seq.token_ids[start:start + n]
            positions += range(start, start + n)
            read = gather_slots(seq.table.block_ids, self.block_size, start + n)
            seq_meta.append((offset, n, read[start:], read))
            count = min(1 + len(seq.draft_token_ids), n)
            rows.append((len(want), count))
            want += range(offset + n - count, offset + n)
        self.last_batch = (token_ids, positions, seq_meta, want)
        logits = self.model.forward(np.asarray(token_ids, dtype=np.int64),
                                    np.asarray(positions, dtype=np.int64),
                                    self.cache_k, self.cache_v, seq_meta,
                                    np.asarray(want, dtype=np.int64))
        return logits, rows

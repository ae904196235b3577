"""Configuration dataclasses for the engine, cache, scheduler and model.

Field names, defaults and validation mirror vllmlite/config.py:4-62 so a caller
of the reference builds these objects unchanged. One field changes meaning:
`EngineConfig.backend` (config.py:60, never read by the reference) selects the
model runner, and defaults to "hip", the gfx950 path in this package.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional


@dataclass
class ModelConfig:
    """Decoder shape. head_dim is d_model // n_heads (config.py:16-18)."""

    n_layers: int = 6
    n_heads: int = 8
    n_kv_heads: int = 8
    d_model: int = 512
    d_ff: int = 2048
    vocab_size: int = 261
    max_seq_len: int = 2048
    weights_path: Optional[str] = None
    seed: int = 1337

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads

    def __post_init__(self):
        # same two checks, same order, same exception type (config.py:20-24)
        if self.d_model % self.n_heads:
            raise ValueError("d_model must divide evenly into n_heads")
        if self.n_heads % self.n_kv_heads:
            raise ValueError("n_heads must be a multiple of n_kv_heads for GQA")


@dataclass
class CacheConfig:
    block_size: int = 16
    num_blocks: int = 1024
    enable_prefix_caching: bool = True
    # element type of the K/V cache: "float32" (the reference's), "bfloat16"
    # (half the cache bytes) or "float8_e4m3" (OCP FP8 E4M3, a quarter; values
    # beyond +-448 saturate); K/V rounded to nearest even when written,
    # everything else stays fp32
    kv_dtype: str = "float32"
    # order of the rows inside a cache block: "token" ([slots, Hkv, D], the
    # reference's), or "head" ([blocks, Hkv, block_size, D]: each KV head's
    # rows of a block contiguous; block_size a power of two)
    kv_layout: str = "token"

    def __post_init__(self):
        if self.kv_dtype not in ("float32", "bfloat16", "float8_e4m3"):
            raise ValueError("kv_dtype must be float32, bfloat16 or float8_e4m3")
        if self.kv_layout not in ("token", "head"):
            raise ValueError("kv_layout must be token or head")
        if self.kv_layout == "head" and self.block_size & (self.block_size - 1):
            raise ValueError("a head-major cache needs a power-of-two block_size")

    @property
    def max_cached_tokens(self) -> int:
        return self.block_size * self.num_blocks


@dataclass
class SchedulerConfig:
    max_seqs: int = 32
    max_batched_tokens: int = 2048
    max_waiting: int = 2048
    chunked_prefill: bool = True
    preemption: str = "recompute"
    watermark: float = 0.01

    def __post_init__(self):
        if self.preemption not in ("recompute", "swap"):
            raise ValueError("preemption must be recompute or swap")


@dataclass
class EngineConfig:
    model: ModelConfig = field(default_factory=ModelConfig)
    cache: CacheConfig = field(default_factory=CacheConfig)
    scheduler: SchedulerConfig = field(default_factory=SchedulerConfig)
    # "hip": HipRunner on the current GPU. The NumPy runner of the reference is
    # not shipped here; pass a runner object to LLMEngine to use another one.
    backend: str = "hip"
    hf_model: Optional[str] = None
    device: str = "cuda"

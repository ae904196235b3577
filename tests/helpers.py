"""Shared builders for the CPU engine tests (mirrors tests/test_engine.py:23-54
of the reference: 2 layers, d 64, H4/Hkv2, d_ff 128, max_len 512)."""

from vllmlite_amd.config import CacheConfig, EngineConfig, ModelConfig, SchedulerConfig
from vllmlite_amd.engine import LLMEngine
from vllmlite_amd.request import SamplingParams

from oracle.runner import NumpyRunner

PROMPTS = [
    "the quick brown fox jumps over",
    "a",
    "systems programming is mostly about memory and never about",
    "hello",
]


def small_cfg(block_size=16, num_blocks=512, max_seqs=8, max_batched=1024,
              prefix_cache=False, chunked=True, layers=2, d_model=64):
    return EngineConfig(
        model=ModelConfig(n_layers=layers, n_heads=4, n_kv_heads=2, d_model=d_model,
                          d_ff=128, max_seq_len=512),
        cache=CacheConfig(block_size=block_size, num_blocks=num_blocks,
                          enable_prefix_caching=prefix_cache),
        scheduler=SchedulerConfig(max_seqs=max_seqs, max_batched_tokens=max_batched,
                                  chunked_prefill=chunked),
    )


def build(runner_factory=None, **kw):
    cfg = small_cfg(**kw)
    factory = runner_factory or NumpyRunner
    return LLMEngine(cfg, runner=factory(cfg.model, cfg.cache))


def run(engine, prompts, max_tokens=20, check_counts=False):
    p = SamplingParams(max_tokens=max_tokens, temperature=0.0, ignore_eos=True)
    ids = [engine.add_request(x, p) for x in prompts]
    while engine.has_work:
        engine.step()
        if check_counts:
            assert engine.batcher.pool.audit()
    return [engine.seqs[i].output_token_ids for i in ids]


def cfg0_config(prefix_cache=False):
    mc = ModelConfig(n_layers=6, n_heads=8, n_kv_heads=4, d_model=384, d_ff=1024,
                     vocab_size=261, max_seq_len=512)
    cc = CacheConfig(block_size=16, num_blocks=512, enable_prefix_caching=prefix_cache)
    return EngineConfig(model=mc, cache=cc,
                        scheduler=SchedulerConfig(max_seqs=16, max_batched_tokens=1024))

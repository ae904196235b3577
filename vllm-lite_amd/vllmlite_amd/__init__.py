"""MI355X-native ragged paged-attention step for vllm-lite.

Host side: the reference's caller interface restated (config, sequence, block,
block_manager, scheduler, engine, sampling, speculative, tokenizer) and the
`HipRunner` that implements the `ModelRunner` boundary on gfx950 through the
C-ABI library built from ../csrc (see `ops`).
"""

__all__ = ["__version__"]
__version__ = "0.1.0"

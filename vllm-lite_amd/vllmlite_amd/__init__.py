"""MI355X-native ragged paged-attention step for vllm-lite.

Host side: `HipRunner` (`hip_runner`), which implements the reference's
`ModelRunner` boundary on gfx950 through the C-ABI library built from ../csrc
(bound by `ops`), and a caller of this package's own design that drives it
end to end with the reference's observable behaviour: `config`, `request`,
`kvpool` (block pool and prefix index), `batcher` (continuous batching),
`engine` (with a one-step lookahead), `sampling`, `speculative`,
`tokenizer`, `model` (weights and RoPE tables), `workload` and `synthetic`
(the benchmark inputs).
"""

__all__ = ["__version__"]
__version__ = "0.1.0"

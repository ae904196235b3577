"""CPU oracle for the ragged paged-attention step. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import
this package, and only as the checker (or, for the baseline, as the timed CPU
path). The product package never imports it.

Contents, each citing the reference file:line it restates:
  attention.py  build_rope, apply_rope, gather_slots, write_kv, softmax,
                paged_attention                     (vllmlite/attention.py:21-98)
  model.py      rms_norm, silu, seeded weights, forward (vllmlite/model.py:17-120)
  runner.py     NumpyRunner: KV cache, CoW, flattening (vllmlite/runner.py:35-100)
  greedy.py     verify / greedy argmax               (vllmlite/speculative.py:86-100,
                                                      vllmlite/sampling.py:56-57)
  dense.py      the textbook dense attention checker (tests/test_attention.py:13-30)

How each function is pinned (tests/test_oracle_*.py):
  gather_slots / write_kv / CoW: the known answer [12,13,14,15,0,1]
      (tests/test_attention.py:60-62) plus brute force on tiny tables.
  paged_attention: the dense checker over the reference's 27-case grid at
      rtol 1e-4 / atol 1e-5 (tests/test_attention.py:33-57), plus closed forms
      (one key -> output equals V; equal keys -> output is the mean of V).
  apply_rope / build_rope: position-0 identity and position dependence
      (tests/test_attention.py:65-77), norm preservation, and a 2x2 rotation
      built independently with math.cos/math.sin.
  rms_norm / silu: closed forms (tests/test_oracle_model.py: a known answer,
      unit RMS, scale invariance, the eps term, silu(0)=0, silu(1), the
      odd-part identity silu(x) - silu(-x) = x).
  verify: the reference's known answers (tests/test_speculative.py:36-60).
  the package's workload generator + the caller side: the published totals 3025/3179 tokens and 260 steps
      (results/mixed_lengths.json:22-23,88) and 14480/3323, 281/280 steps
      (results/shared_prefix.json).
  forward / seeded weights / end-to-end greedy streams: golden fixtures written
      by tests/golden/make_golden.py from the reference itself.
"""

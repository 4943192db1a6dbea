"""CPU oracle for the speculative-decoding verification path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (`adaptive-specdec_amd/`)
imports, links or runs anything in this directory; only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` use it, and
only as the checker (or, for the baseline, as the CPU program being timed).

It is a numpy restatement of the reference's hot path:

* `specdec/sampling.py:34-95` (`to_probs`, `sample_from_probs`,
  `residual_probs`, `gather_prob`) -> `oracle.sampling`
* `specdec/engine.py:281-312` (accept loop, residual/bonus draw, rollback
  counts) -> `oracle.sampling.rejection_sample`
* `specdec/kvcache.py:53-190` (ragged scatter, lengths, rollback, mask) and the
  paged slot formula of `vllm_draft_spec/proposer.py:295-314` -> `oracle.kvcache`
* `specdec/controller.py:47-67` (closed-form k choice) -> `oracle.controller`
* verify attention (HF SDPA over the ragged cache) -> `oracle.attention`

Where the reference leaves the arithmetic to torch internals that differ by
ISA, thread count and device (softmax's exp and fp32 sum order, the unstable
CPU sort, multinomial's internal noise stream), the oracle fixes one
deterministic rule, documented in `oracle/numerics.py` and at each function.
"""

"""specdec on MI355X: the speculative-decoding verification path as HIP kernels.

Drop-in for the reference package's hot path:
  specdec.sampling      to_probs, sample_from_probs, residual_probs, gather_prob,
                        rejection_sample
  specdec.kvcache       RaggedCache (+ PagedKVCache for the shared-block-table layout)
  specdec.proposer_ops  greedy_draft_tokens, drafting_slot_mapping
  specdec.controller    expected_speedup, best_k
The native library (libspecdec_amd.so) is loaded on first use.
"""
__version__ = "0.1.0"

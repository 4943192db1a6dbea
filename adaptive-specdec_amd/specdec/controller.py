"""Closed-form draft length (`specdec/controller.py:47-67`), host side.

The expected tokens per round of Leviathan et al., (1 - a^(k+1)) / (1 - a),
over the cost of the round in target forwards, (k + x) c + 1, where x is the
number of draft forwards a round costs beyond k (1 for the from-scratch engine,
0 for the vLLM proposer, `vllm_draft_spec/proposer.py:89`). The verify path
uses it to pick a per-row k; it is scalar host work, not a kernel.
"""

__all__ = ["expected_speedup", "best_k", "best_k_rows"]


def expected_speedup(k, alpha, c, extra_fwd=1):
    """Expected tokens per round divided by the round's cost (`controller.py:47-61`)."""
    k = max(1, int(k))
    if alpha >= 1.0 - 1e-9:
        tokens = float(k + 1)
    else:
        tokens = (1.0 - alpha ** (k + 1)) / (1.0 - alpha)
    return tokens / ((k + extra_fwd) * c + 1.0)


def best_k(alpha, c, k_max=8, extra_fwd=1):
    """argmax over k in [1, k_max] (`controller.py:64-67`); the smallest k wins ties."""
    return max(range(1, int(k_max) + 1), key=lambda k: expected_speedup(k, alpha, c, extra_fwd))


def best_k_rows(alphas, c, k_max=8, extra_fwd=1):
    """best_k for each row's acceptance estimate (a list of per-row k)."""
    return [best_k(float(a), c, k_max, extra_fwd) for a in alphas]

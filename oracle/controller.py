"""Oracle restatement of the closed-form draft-length rule, `specdec/controller.py:47-67`.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`).
"""


def expected_speedup(k, alpha, c, extra_fwd=1):
    """(1 - a^(k+1)) / ((1 - a) * ((k + x) c + 1)), with the a -> 1 limit k + 1."""
    k = max(1, int(k))
    tokens = float(k + 1) if alpha >= 1.0 - 1e-9 else (1.0 - alpha ** (k + 1)) / (1.0 - alpha)
    return tokens / ((k + extra_fwd) * c + 1.0)


def best_k(alpha, c, k_max=8, extra_fwd=1):
    """argmax over k in [1, k_max]; the first (smallest) k wins ties, as `max` does."""
    best, best_v = 1, None
    for k in range(1, int(k_max) + 1):
        v = expected_speedup(k, alpha, c, extra_fwd)
        if best_v is None or v > best_v:
            best, best_v = k, v
    return best

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


class EWMAState:
    """`EWMAAnalytic` (`controller.py:121-154`): alpha = accepted / positions
    reached with a per-token decay beta^reached, an EWMA of c, warmup rounds at
    k_init, then best_k."""

    def __init__(self, k_max=8, beta=0.99, k_init=4, c_init=0.15, warmup=3, extra_fwd=1):
        self.k_max, self.beta, self.k_init = int(k_max), float(beta), int(k_init)
        self.c, self.warmup, self.extra_fwd = float(c_init), int(warmup), int(extra_fwd)
        self.acc = 0.0
        self.reached = 0.0
        self.rounds = 0
        self.last_k = self.k_init

    @property
    def alpha(self):
        if self.reached <= 0:
            return 0.7
        return min(0.999, max(0.0, self.acc / self.reached))

    def propose_k(self):
        """`controller.py:136-141`."""
        if self.rounds < self.warmup:
            self.last_k = self.k_init
        else:
            self.last_k = best_k(self.alpha, self.c, self.k_max, self.extra_fwd)
        return self.last_k

    def update(self, k, n_accepted, c_obs=None):
        """`controller.py:143-154` (c_obs stands for t_draft_fwd / t_target_fwd)."""
        acc = float(sum(int(a) for a in n_accepted))
        reached = float(sum(min(int(a) + 1, int(k)) for a in n_accepted))
        w = self.beta ** reached
        self.acc = w * self.acc + acc
        self.reached = w * self.reached + reached
        if c_obs is not None and c_obs > 0:
            self.c = 0.9 * self.c + 0.1 * float(c_obs)
        self.rounds += 1

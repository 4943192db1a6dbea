"""Gate G1 on the oracle: speculative sampling must reproduce the target distribution.

Re-creates the reference's statistical test (`tests/test_rejection_sampling.py:64-126`,
gate `config.py:72` G1_TV_MAX = 0.02) and the enumerable-vocab workload
B=1, k=4, V=64 (target ~ N(0, 2^2), draft = target + N(0, 0.8^2), T = 1,
100,000 seeded trials). The negative controls plant their bugs in a copy of
the oracle's accept rule, on the CPU, and must be caught.
"""
import numpy as np
import pytest

from oracle import sampling as S
from oracle.numerics import fixed62, uniform_threshold

G1_TV_MAX = 0.02


def uniforms(rs, shape):
    """fp32 uniforms in [0, 1) on the 2**-24 grid (the form torch.rand returns)."""
    return (rs.randint(0, 1 << 24, size=shape).astype(np.float64) * 2.0 ** -24).astype(np.float32)


class Dist:
    """A fixed distribution prepared for repeated inverse-CDF draws."""

    def __init__(self, w):
        self.w = np.asarray(w, np.uint64)
        self.cum = np.cumsum(self.w, dtype=np.uint64)
        self.tot = int(self.cum[-1])

    def draw(self, u):
        return int(np.searchsorted(self.cum, np.uint64(uniform_threshold(u, self.tot)), side="right"))


def simulate(P, Q, ud, ua, uf, mode="correct"):
    """One speculative round per trial on fixed per-position distributions.

    P [k+1, V], Q [k, V] fp32 probs. Returns (n_acc [N], first emitted token [N]).
    Draft tokens x_i ~ Q_i by inverse CDF on ud; accept/residual as the oracle.
    """
    k = Q.shape[0]
    qd = [Dist(fixed62(Q[i])) for i in range(k)]
    res = [Dist(S._residual_weights(P[i], Q[i])) for i in range(k)]
    pd = [Dist(fixed62(P[i])) for i in range(k + 1)]
    N = ud.shape[0]
    n_out = np.zeros(N, np.int64)
    first = np.zeros(N, np.int64)
    for t in range(N):
        xs = [qd[i].draw(ud[t, i]) for i in range(k)]
        if mode == "always_accept":
            n = k
        else:
            n, _ = S.accept_chain(P[np.arange(k), xs], Q[np.arange(k), xs], ua[t], True)
        if n == k:
            y = pd[k].draw(uf[t])
        elif mode == "resample_from_p":
            y = pd[n].draw(uf[t])
        else:
            y = res[n].draw(uf[t])
        n_out[t] = n
        first[t] = xs[0] if n >= 1 else y
    return n_out, first


def tv(a, b):
    return 0.5 * float(np.abs(a - b).sum())


def empirical(ids, V):
    return np.bincount(ids, minlength=V) / len(ids)


@pytest.fixture(scope="module")
def config1():
    rs = np.random.RandomState(20241)
    k, V, N = 4, 64, 100_000
    tgt = (rs.randn(k + 1, V) * 2.0).astype(np.float32)
    drf = (tgt[:k] + rs.randn(k, V) * 0.8).astype(np.float32)
    P = S.to_probs(tgt, temperature=1.0)
    Q = S.to_probs(drf, temperature=1.0)
    ud, ua, uf = uniforms(rs, (N, k)), uniforms(rs, (N, k)), uniforms(rs, N)
    return P, Q, ud, ua, uf


def test_g1_config1_lossless(config1):
    P, Q, ud, ua, uf = config1
    k, V = Q.shape
    n, first = simulate(P, Q, ud, ua, uf)
    d = tv(empirical(first, V), P[0])
    floor = (V / (2 * np.pi * len(first))) ** 0.5
    assert d < G1_TV_MAX, f"TV={d:.4f} floor={floor:.4f}"
    # accepted-length histogram against the closed form P(n=a) = prod beta_i (1 - beta_a)
    beta = np.minimum(P[:k].astype(np.float64), Q.astype(np.float64)).sum(-1)
    assert 0.45 < beta.mean() < 0.75
    expect = np.array([np.prod(beta[:a]) * (1 - beta[a]) for a in range(k)] + [np.prod(beta)])
    got = np.bincount(n, minlength=k + 1) / len(n)
    sigma = np.sqrt(expect * (1 - expect) / len(n))
    assert np.all(np.abs(got - expect) < 5 * sigma + 1e-4), (got, expect)


@pytest.mark.parametrize("mode", ["always_accept", "resample_from_p"])
def test_g1_detects_planted_bugs(config1, mode):
    P, Q, ud, ua, uf = config1
    N = 40_000
    _, first = simulate(P, Q, ud[:N], ua[:N], uf[:N], mode=mode)
    assert tv(empirical(first, Q.shape[1]), P[0]) > G1_TV_MAX


def test_g1_part_a_mismatched_top_p():
    """Reference part A (`test_rejection_sampling.py:102-126`): top-p applied with
    a different cutoff on the draft must be detected; the consistent one not."""
    rs = np.random.RandomState(7)
    V, N = 16, 60_000
    lp = (rs.randn(V) * 1.5).astype(np.float32)
    lq = (lp + rs.randn(V) * 0.8).astype(np.float32)
    p = S.to_probs(lp, 1.0, top_p=0.9)
    q_right = S.to_probs(lq, 1.0, top_p=0.9)
    q_bad = S.to_probs(lq, 1.0, top_p=0.5)
    assert float(np.minimum(p, q_right).sum()) > 0.2          # non-degenerate control
    ud, ua, uf = uniforms(rs, (N, 1)), uniforms(rs, (N, 1)), uniforms(rs, N)
    P = np.stack([p, p])
    _, ok_first = simulate(P, q_right[None], ud, ua, uf)
    assert tv(empirical(ok_first, V), p) < 0.015
    # bug: x drawn from the differently truncated q, tested against q_right
    qd = Dist(fixed62(q_bad))
    res = Dist(S._residual_weights(p, q_right))
    bad = []
    for t in range(N):
        x = qd.draw(ud[t, 0])
        n, _ = S.accept_chain(p[[x]], q_right[[x]], ua[t], True)
        bad.append(x if n else res.draw(uf[t]))
    assert tv(empirical(np.array(bad), V), p) > G1_TV_MAX

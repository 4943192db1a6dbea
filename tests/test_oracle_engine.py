"""Pins of the round-level oracle pieces: the draft step (`engine.py:250-258`,
`controller.py:184-187`), EWMAAnalytic's state (`controller.py:121-154`) and the
end-of-round bookkeeping (`engine.py:305-340`), by hand-computed cases, closed
forms and sampling statistics."""
import math

import numpy as np

from oracle import controller as OC
from oracle import engine as OE
from oracle import sampling as OS


def test_draft_step_draws_from_q_and_tracks_conf():
    rng = np.random.default_rng(0)
    V, N = 16, 40000
    row = (rng.standard_normal(V) * 1.5).astype(np.float32)
    q = OS.to_probs(row[None], 0.9, 0.9)[0]
    u = rng.random(N, dtype=np.float32)
    # the draw of every row is the inverse-CDF draw of sample_fixed
    x, qx, conf, stop = OS.draft_step(np.repeat(row[None], 64, 0), u[:64], 0.9, 0.9,
                                      conf=np.ones(64, np.float32), tau=0.5, step=1)
    assert np.array_equal(x, [OS.sample_fixed(OS.fixed62(q), uu) for uu in u[:64]])
    assert np.array_equal(qx, q[x]) and np.array_equal(conf, q[x])
    # the empirical distribution of the draws is q (TV well under the sampling noise)
    cdf = np.cumsum(OS.fixed62(q).astype(object))
    tot = int(cdf[-1])
    xs = np.array([int(np.searchsorted(np.array(cdf, dtype=object), (int(uu * (1 << 24)) * tot) >> 24,
                                        side="right")) for uu in u])
    emp = np.bincount(xs, minlength=V) / N
    assert 0.5 * np.abs(emp - q).sum() < 0.02
    assert np.all(emp[q == 0] == 0)                 # dropped tokens are never drafted


def test_draft_step_early_exit_threshold():
    logits = np.array([[0.0, 0.0], [3.0, 0.0]], np.float32)      # q(x) = 0.5, then ~0.95
    u = np.array([0.25, 0.5], np.float32)
    x, qx, conf, stop = OS.draft_step(logits, u, 1.0, conf=np.array([0.6, 0.2], np.float32),
                                      tau=0.3, step=2, min_k=1)
    assert x.tolist() == [0, 0] and qx[0] == np.float32(0.5)
    assert conf[0] == np.float32(0.3) and conf[1] == np.float32(np.float32(0.2) * qx[1])
    mean = np.float32(np.float32(conf[0] + conf[1]) / np.float32(2))
    assert stop == int(mean < np.float32(0.3))
    # before min_k the test never stops the loop
    _, _, _, stop = OS.draft_step(logits, u, 1.0, conf=np.zeros(2, np.float32), tau=0.3, step=1,
                                  min_k=2)
    assert stop == 0
    # greedy: the first argmax, probability 1, conf unchanged
    x, qx, conf, _ = OS.draft_step(np.array([[1.0, 5.0, 5.0]], np.float32), None, 0.0,
                                   conf=np.array([0.7], np.float32))
    assert x.tolist() == [1] and qx[0] == 1.0 and conf[0] == np.float32(0.7)


def test_ewma_state_closed_form():
    c = OC.EWMAState(k_max=8, beta=0.9, k_init=3, c_init=0.2, warmup=2)
    assert c.propose_k() == 3 and c.alpha == 0.7
    # round 1 at k=4: rows accept 4, 0, 2 -> accepted 6, reached 4 + 1 + 3 = 8
    c.update(4, [4, 0, 2])
    assert c.acc == 6.0 and c.reached == 8.0 and c.rounds == 1
    assert c.propose_k() == 3                         # still warming up
    # round 2 at k=3: accepted 1 + 3 = 4, reached 2 + 3 = 5, decay 0.9^5 on the old sums
    c.update(3, [1, 3], c_obs=0.4)
    w = 0.9 ** 5
    assert math.isclose(c.acc, w * 6 + 4, rel_tol=0, abs_tol=1e-15)
    assert math.isclose(c.reached, w * 8 + 5, rel_tol=0, abs_tol=1e-15)
    assert math.isclose(c.c, 0.9 * 0.2 + 0.1 * 0.4, abs_tol=1e-15)
    assert c.propose_k() == OC.best_k(c.alpha, c.c, 8, 1)
    # beta = 1: alpha is the plain ratio of totals; the estimate is clamped at 0.999
    d = OC.EWMAState(beta=1.0, warmup=0)
    for n in ([2, 2], [1, 0], [3]):
        d.update(3, n)
    assert d.alpha == (2 + 2 + 1 + 0 + 3) / (3 + 3 + 2 + 1 + 3)
    e = OC.EWMAState(warmup=0)
    e.update(2, [2, 2, 2])
    assert e.alpha == 0.999


def test_round_commit_cases():
    eos = [7]
    out = [[5], [5], [5], [5]]
    # row 0: 2 of 3 accepted then y; row 1: an accepted EOS ends it before y;
    # row 2: already done; row 3: reaches max_new inside its accepted drafts
    drop, done, out = OE.round_commit(n_acc=[2, 3, 1, 3], y=[9, 9, 9, 9],
                                      draft_ids=[[1, 2, 3], [4, 7, 8], [1, 1, 1], [1, 2, 3]], k=3,
                                      done=[False, False, True, False], out=out, eos_ids=eos,
                                      max_new=3)
    assert drop.tolist() == [1, 0, 2, 0]
    assert out == [[5, 1, 2], [5, 4, 7], [5], [5, 1, 2]]
    assert done.tolist() == [True, True, True, True]
    out = [[5], [5]]
    drop, done, out = OE.round_commit([0, 1], [7, 8], [[1, 2], [3, 4]], 2, [False, False], out,
                                      eos, 10)
    assert out == [[5, 7], [5, 3, 8]] and done.tolist() == [True, False] and drop.tolist() == [2, 1]
    # per-row k: packed drafts at cu_k
    out = [[0], [0]]
    drop, done, out = OE.round_commit([1, 0], [9, 9], [4, 5, 6], None, [False, False], out, eos,
                                      10, cu_k=[0, 2, 3])
    assert out == [[0, 4, 9], [0, 9]] and drop.tolist() == [1, 1]

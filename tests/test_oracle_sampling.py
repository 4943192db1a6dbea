"""Pins for `oracle/sampling.py` (restating `specdec/sampling.py:34-95` and
`specdec/engine.py:281-303`).

* Known answers, computed by hand on dyadic probabilities where fp32 is exact.
* Closed forms: T = 0 one-hot (first index), top_p = 1 & top_k = 0 softmax
  against float64 numpy, sum to one.
* Brute force: the fp32 nucleus rule against the exact-rational nucleus on
  random rows, wherever the rounding margin is wider than 1e-6.
* A cross-check against torch's own CPU softmax/topk/sort/cumsum (the ops the
  reference calls), probabilities within 1e-5 absolute.
* Accept-loop and sampler invariants against brute force.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import sampling as S
from oracle.numerics import fixed62, rn32


def f32(*v):
    return np.array(v, np.float32)


# ---------------------------------------------------------------- known answers
def test_kat_uniform_softmax():
    out = S.to_probs(np.zeros((2, 4), np.float32), temperature=0.7)
    assert np.array_equal(out, np.full((2, 4), 0.25, np.float32))


def test_kat_masked_token():
    out = S.to_probs(f32(0.0, -np.inf, 0.0, 0.0), temperature=1.0)
    third = np.float32(1.0) / np.float32(3.0)
    assert out[1] == 0.0
    assert np.allclose(out[[0, 2, 3]], third, rtol=0, atol=1e-7)


@pytest.mark.parametrize("T", [0.0, -1.0, None])
def test_kat_greedy_first_index(T):
    out = S.to_probs(f32(1.0, 3.0, 3.0, 2.0), temperature=T, top_p=0.5, top_k=2)
    assert np.array_equal(out, f32(0, 1, 0, 0))


P4 = f32(0.125, 0.5, 0.125, 0.25)   # sorted: id1 0.5, id3 0.25, id0 0.125, id2 0.125


@pytest.mark.parametrize("top_p,top_k,expect", [
    (0.5, None, f32(0, 1, 0, 0)),                       # cum-srt = 0, .5, .75, .875
    (0.6, None, f32(0, 2 / 3, 0, 1 / 3)),
    (0.8, None, f32(1 / 7, 4 / 7, 0, 2 / 7)),           # tie 0.125: id0 kept, id2 dropped
    (0.9, None, f32(0.125, 0.5, 0.125, 0.25)),          # .875 < .9: all four kept
    (None, 2, f32(0, 2 / 3, 0, 1 / 3)),                 # kth = 0.25
    (None, 3, f32(0.125, 0.5, 0.125, 0.25)),            # kth = 0.125: ties at kth survive
    (0.8, 3, f32(1 / 7, 4 / 7, 0, 2 / 7)),
])
def test_kat_filters(top_p, top_k, expect):
    got = S.filter_renorm(P4.copy(), top_p, top_k)
    assert np.array_equal(got, expect), (got, expect)


def test_kat_top_p_uses_unrenormalised_top_k_mass():
    # sampling.py:52-64 applies top-p to the top-k-zeroed probs WITHOUT
    # renormalising: mass of {0.5, 0.25} is 0.75, so at top_p=0.6 the second
    # token's exclusive mass is 0.5 < 0.6 and it survives. (Renormalising first
    # would give 2/3 > 0.6 and drop it.)
    got = S.filter_renorm(f32(0.5, 0.25, 0.125, 0.125), top_p=0.6, top_k=2)
    assert np.array_equal(got, f32(2 / 3, 1 / 3, 0, 0))


def test_kat_tie_group_keeps_lowest_ids():
    # eight equal tokens: the nucleus boundary falls inside the tie group; the
    # stable rule keeps the lowest token ids.
    p = np.full(8, 0.125, np.float32)
    got = S.filter_renorm(p, top_p=0.3)          # excl. mass 0, .125, .25 < .3; .375 not
    assert np.array_equal(got, f32(1 / 3, 1 / 3, 1 / 3, 0, 0, 0, 0, 0))


# ---------------------------------------------------------------- closed forms
def test_softmax_matches_float64():
    rs = np.random.RandomState(0)
    x = (rs.randn(16, 997) * 3).astype(np.float32)
    for T in (0.3, 0.8, 1.0, 2.5):
        got = S.to_probs(x, temperature=T)
        s = x / np.float32(T)
        d = (s - s.max(-1, keepdims=True)).astype(np.float64)   # fp32 `x - max`, as softmax does
        ref = np.exp(d)
        ref /= ref.sum(-1, keepdims=True)
        assert np.max(np.abs(got - ref) / ref) < 1e-6
        exact = np.exp(s.astype(np.float64) - s.max(-1, keepdims=True))
        exact /= exact.sum(-1, keepdims=True)
        assert np.max(np.abs(got - exact)) < 1e-7
        assert np.max(np.abs(got.astype(np.float64).sum(-1) - 1)) < 1e-6


def test_filtered_rows_sum_to_one_and_keep_mass():
    rs = np.random.RandomState(1)
    for _ in range(40):
        V = int(rs.randint(8, 300))
        x = (rs.randn(V) * 3).astype(np.float32)
        T = float(rs.uniform(0.3, 1.5))
        tp = float(rs.uniform(0.05, 0.99))
        tk = int(rs.randint(0, V))
        raw = S.to_probs(x, temperature=T)
        out = S.to_probs(x, temperature=T, top_p=tp, top_k=tk)
        kept = out > 0
        assert abs(float(out.astype(np.float64).sum()) - 1) < 1e-6
        kept_mass = float(raw[kept].astype(np.float64).sum())
        # nucleus holds at least top_p of the (top-k) mass unless everything is kept
        if tk and tk < V:
            kth = np.sort(raw)[-tk]
            topk_mass = float(raw[raw >= kth].astype(np.float64).sum())
            assert kept_mass >= min(tp, topk_mass) - 1e-6
        else:
            assert kept_mass >= tp - 1e-6


# ---------------------------------------------------------------- brute force
def _exact_nucleus(p, tp):
    """Exact-rational nucleus: in stable descending order keep a token iff the
    exact mass strictly before it is < top_p (first token always kept).
    Returns (mask, min_margin)."""
    order = sorted(range(len(p)), key=lambda i: (-float(p[i]), i))
    tpe = Fraction(float(np.float32(tp)))
    mass = Fraction(0)
    keep = np.zeros(len(p), bool)
    margin = None
    for rank, i in enumerate(order):
        gap = abs(float(mass - tpe))
        margin = gap if margin is None else min(margin, gap)
        keep[i] = rank == 0 or mass < tpe
        mass += Fraction(float(p[i]))
    return keep, margin


def test_nucleus_matches_exact_rational():
    rs = np.random.RandomState(2)
    checked = 0
    for _ in range(300):
        V = int(rs.randint(4, 64))
        # bf16-like logits so that ties occur
        x = torch.tensor(rs.randn(V) * 2, dtype=torch.bfloat16).float().numpy()
        tp = float(rs.uniform(0.05, 0.99))
        raw = S.to_probs(x, temperature=1.0)
        got = S.filter_renorm(raw.copy(), top_p=tp) > 0
        exact, margin = _exact_nucleus(raw, tp)
        if margin > 1e-6:
            assert np.array_equal(got, exact)
            checked += 1
    assert checked > 250


# ---------------------------------------------------------------- torch cross-check
def _torch_to_probs(logits, temperature, top_p, top_k):
    """The op sequence of `sampling.py:42-67`, run with torch's own CPU kernels
    (stable sort so tie order is comparable)."""
    logits = logits.float()
    probs = torch.softmax(logits / temperature, dim=-1)
    if top_k and 0 < top_k < probs.shape[-1]:
        kth = probs.topk(top_k, dim=-1).values[..., -1:]
        probs = torch.where(probs < kth, torch.zeros_like(probs), probs)
    if top_p is not None and 0.0 < top_p < 1.0:
        srt, idx = torch.sort(probs, dim=-1, descending=True, stable=True)
        cum = srt.cumsum(dim=-1)
        keep = cum - srt < top_p
        keep[..., 0] = True
        mask = torch.zeros_like(probs, dtype=torch.bool).scatter_(-1, idx, keep)
        probs = torch.where(mask, probs, torch.zeros_like(probs))
    return probs / probs.sum(dim=-1, keepdim=True).clamp_min(1e-12)


@pytest.mark.parametrize("T,tp,tk", [(0.8, 0.95, 0), (0.7, 0.9, 50), (1.0, 1.0, 0), (1.3, 0.5, 7)])
def test_matches_torch_cpu_ops(T, tp, tk):
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(12, 4096, generator=g) * 3).to(torch.bfloat16)
    ref = _torch_to_probs(x, T, tp, tk).numpy()
    got = S.to_probs(x.float().numpy(), temperature=T, top_p=tp, top_k=tk)
    assert np.max(np.abs(got - ref)) < 1e-5
    # kept sets agree except possibly at one boundary tie group per row
    diff_rows = np.nonzero(((got > 0) != (ref > 0)).any(-1))[0]
    for r in diff_rows:
        d = np.nonzero((got[r] > 0) != (ref[r] > 0))[0]
        vals = x[r].float().numpy()[d]
        assert np.all(vals == vals[0])            # all in one bf16 tie group


# ---------------------------------------------------------------- sampler / accept
def test_sample_fixed_brute_force():
    rs = np.random.RandomState(4)
    for _ in range(200):
        V = int(rs.randint(1, 40))
        p = rs.dirichlet(np.ones(V)).astype(np.float32)
        p[rs.rand(V) < 0.3] = 0
        w = fixed62(p)
        if int(w.astype(object).sum()) == 0:
            assert S.sample_fixed(w, np.float32(0.3)) == -1
            continue
        u = np.float32(rs.uniform())
        tot = sum(int(v) for v in w)
        t = (Fraction(float(u)) * tot).__floor__()
        run, want = 0, None
        for j, v in enumerate(w):
            run += int(v)
            if run > t:
                want = j
                break
        assert S.sample_fixed(w, u) == want
        assert w[want] > 0


def test_accept_chain_brute_force():
    rs = np.random.RandomState(5)
    for _ in range(500):
        k = int(rs.randint(1, 9))
        px = rs.uniform(0, 1, k).astype(np.float32)
        qx = rs.uniform(0, 1, k).astype(np.float32)
        qx[rs.rand(k) < 0.1] = 0
        u = rs.uniform(0, 1, k).astype(np.float32)
        alive = bool(rs.rand() < 0.9)
        n, _ = S.accept_chain(px, qx, u, alive)
        want = 0
        if alive:
            for i in range(k):
                r = float(px[i]) / max(float(qx[i]), float(np.float32(1e-10)))
                if float(u[i]) < min(r, 1.0):
                    want += 1
                else:
                    break
        assert n == want


def test_rejection_sample_greedy_equals_greedy_verify():
    rs = np.random.RandomState(6)
    B, k, V = 6, 4, 50
    tl = torch.tensor(rs.randn(B, k + 1, V), dtype=torch.bfloat16).float().numpy()
    dl = tl[:, :k] + rs.randn(B, k, V).astype(np.float32) * 0.5
    am = tl[:, :k].argmax(-1)
    ids = np.where(rs.rand(B, k) < 0.6, am, (am + 1) % V)
    ua = rs.uniform(0, 1, (B, k)).astype(np.float32)
    uf = rs.uniform(0, 1, B).astype(np.float32)
    a = S.rejection_sample(tl, dl, ids, ua, uf, temperature=0.0)
    b = S.greedy_verify(tl, ids, ua)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_residual_probs_degenerate_is_p():
    p = f32(0, 1, 0, 0)
    assert np.array_equal(S.residual_probs(p, p), p)
    out = S.residual_probs(f32(0.5, 0.5, 0, 0), f32(0.25, 0.75, 0, 0))
    assert np.array_equal(out, f32(1, 0, 0, 0))


# ---------------------------------------------------------------- per-row k
@pytest.mark.parametrize("T,tp,tk", [(0.8, 0.95, 0), (0.7, 0.9, 5), (0.0, 1.0, 0)])
def test_ragged_with_equal_k_is_the_uniform_verify(T, tp, tk):
    """Packing [B, k+1, V] / [B, k, V] row by row with cu_k = k * arange(B+1)
    must give exactly the uniform-k verify."""
    rs = np.random.RandomState(9)
    B, k, V = 5, 3, 40
    tl = torch.tensor(rs.randn(B, k + 1, V) * 2, dtype=torch.bfloat16).float().numpy()
    dl = torch.tensor(tl[:, :k] + rs.randn(B, k, V), dtype=torch.bfloat16).float().numpy()
    ids = rs.randint(0, V, (B, k))
    ua = rs.uniform(0, 1, (B, k)).astype(np.float32)
    uf = rs.uniform(0, 1, B).astype(np.float32)
    want = S.rejection_sample(tl, dl, ids, ua, uf, T, tp, tk)
    got = S.rejection_sample_ragged(tl.reshape(-1, V), dl.reshape(-1, V), ids.reshape(-1),
                                    ua.reshape(-1), uf, np.arange(B + 1) * k, T, tp, tk)
    for x, y in zip(got, want):
        assert np.array_equal(x, y)


def test_ragged_rows_use_their_own_slices():
    """Rows of k_b = 2, 0, 3: each equals the uniform verify of that row alone
    on its packed slices, and the k_b = 0 row emits the bonus draw of its one
    target row (to_probs then the fixed-point inverse CDF)."""
    rs = np.random.RandomState(10)
    V, ks = 32, [2, 0, 3]
    cu = np.concatenate([[0], np.cumsum(ks)])
    nt, nd = sum(ks) + len(ks), sum(ks)
    tl = torch.tensor(rs.randn(nt, V) * 2, dtype=torch.bfloat16).float().numpy()
    dl = torch.tensor(rs.randn(nd, V) * 2, dtype=torch.bfloat16).float().numpy()
    ids = rs.randint(0, V, nd)
    ua = rs.uniform(0, 1, nd).astype(np.float32)
    uf = rs.uniform(0, 1, len(ks)).astype(np.float32)
    n, y, f = S.rejection_sample_ragged(tl, dl, ids, ua, uf, cu, 0.9, 0.9, 0)
    for b, kb in enumerate(ks):
        c0 = int(cu[b])
        if kb == 0:
            p = S.to_probs(tl[c0 + b][None], 0.9, 0.9, 0)
            assert n[b] == 0 and y[b] == S.sample_from_probs(p, uf[b:b + 1])[0]
            continue
        rn, ry, rf = S.rejection_sample(tl[None, c0 + b:c0 + b + kb + 1], dl[None, c0:c0 + kb],
                                        ids[None, c0:c0 + kb], ua[None, c0:c0 + kb], uf[b:b + 1],
                                        0.9, 0.9, 0)
        assert (n[b], y[b], f[b]) == (rn[0], ry[0], rf[0])


# ---------------------------------------------------------------- tie-order flag
def _kept_under_order(p, top_p, rank):
    """The nucleus of `sampling.py:57-64` when equal probabilities are sorted by
    `rank` (any tie order the unstable sort may produce): the kept ids."""
    order = sorted(range(p.size), key=lambda i: (-float(p[i]), rank[i]))
    srt = p[order]
    cum = np.cumsum(fixed62(srt), dtype=np.uint64)
    kept = set()
    for j, i in enumerate(order):
        excl = rn32(int(cum[j])) - srt[j]
        if j == 0 or excl < np.float32(top_p):
            kept.add(i)
    return kept


def _softmax_topk(x, T, tk):
    p = S._softmax_row(np.asarray(x, np.float32), T)
    if tk:
        kth = np.sort(p)[-tk]
        p = np.where(p < kth, np.float32(0.0), p)
    return p


def test_kat_boundary_tie_group():
    """A planted group of four equal logits with the cut after two of them is
    the group; a cut after all four (or top_p off, or greedy) gives none."""
    x = np.array([3.0, 2.0, 1.0, 2.0, 0.5, 2.0, 2.0, -1.0], np.float32)
    p = S._softmax_row(x, 1.0)
    m3, p2 = float(p[0]), float(p[1])
    g = S.boundary_tie_group(x, 1.0, m3 + 1.5 * p2, 0)
    assert g is not None and g.tolist() == (x == 2.0).tolist()
    assert S.boundary_tie_group(x, 1.0, m3 + 3.5 * p2, 0) is None
    assert S.boundary_tie_group(x, 1.0, 1.0, 0) is None
    assert S.boundary_tie_group(x, 0.0, m3 + 1.5 * p2, 0) is None


def test_boundary_tie_group_is_what_the_tie_order_decides():
    """Brute force on tie-heavy rows: the group is exactly the set of ids whose
    membership in the nucleus changes with the order of equal probabilities."""
    rng = np.random.default_rng(12)
    n_partial = 0
    for trial in range(150):
        V = int(rng.integers(4, 24))
        x = rng.integers(0, 5, V).astype(np.float32) * np.float32(0.75)
        T = float(rng.choice([0.5, 1.0, 1.7]))
        tp = float(rng.uniform(0.2, 0.97))
        tk = int(rng.integers(0, V)) if trial % 3 == 0 else 0
        p = _softmax_topk(x, T, tk)
        kept = [_kept_under_order(p, tp, rng.permutation(V)) for _ in range(120)]
        kept.append(_kept_under_order(p, tp, np.arange(V)))
        varies = np.array([len({i in k for k in kept}) == 2 for i in range(V)])
        g = S.boundary_tie_group(x, T, tp, tk)
        if g is None:
            assert not varies.any(), trial
        else:
            n_partial += 1
            assert np.array_equal(g, varies), trial
            # the oracle's own nucleus is the lowest-ids-first order
            probs = S._transform_row(x, T, tp, tk)
            assert set(np.nonzero(probs > 0)[0].tolist()) == kept[-1]
    assert n_partial > 20


def _rs_with_order(tl, dl, ids, ua, uf, T, tp, tk, rank_of):
    """rejection_sample with the nucleus taken under tie orders rank_of(row)."""
    def probs(x, r):
        p = _softmax_topk(x, T, tk)
        keep = _kept_under_order(p, tp, r)
        q = np.array([p[i] if i in keep else 0.0 for i in range(p.size)], np.float32)
        tot = max(rn32(sum(int(v) for v in fixed62(q))), np.float32(1e-12))
        return (q / tot).astype(np.float32)
    B, k1, V = tl.shape
    k = k1 - 1
    n_acc = np.zeros(B, np.int64)
    for b in range(B):
        px = [probs(tl[b, i], rank_of(b, i))[ids[b, i]] for i in range(k)]
        qx = [probs(dl[b, i], rank_of(b, 100 + i))[ids[b, i]] for i in range(k)]
        n_acc[b], _ = S.accept_chain(np.array(px, np.float32), np.array(qx, np.float32), ua[b], True)
    return n_acc


def test_tie_order_flag_covers_every_order_dependent_accept():
    """Rows whose accepted count changes under another order of equal values in
    the sort are flagged; rows without partial groups never are."""
    rng = np.random.default_rng(5)
    B, k, V = 24, 3, 16
    T, tp, tk = 1.0, 0.6, 0
    tl = (rng.integers(0, 4, (B, k + 1, V)) * 0.5).astype(np.float32)
    dl = (tl[:, :k] + (rng.integers(0, 2, (B, k, V)) * 0.5)).astype(np.float32)
    ids = np.zeros((B, k), np.int64)
    for b in range(B):
        for i in range(k):
            g = S.boundary_tie_group(dl[b, i], T, tp, tk)
            pool = np.nonzero(g)[0] if g is not None and rng.random() < 0.7 else np.arange(V)
            ids[b, i] = int(rng.choice(pool))
    ua = rng.random((B, k)).astype(np.float32)
    uf = rng.random(B).astype(np.float32)
    n, y, fl = S.rejection_sample(tl, dl, ids, ua, uf, T, tp, tk)
    tied = (fl & S.FLAG_TIE_ORDER) != 0
    assert tied.any() and not tied.all()
    for seed in range(25):
        r = np.random.default_rng(100 + seed)
        perms = {}

        def rank_of(b, i):
            return perms.setdefault((b, i), r.permutation(V))
        n2 = _rs_with_order(tl, dl, ids, ua, uf, T, tp, tk, rank_of)
        assert np.all(tied | (n2 == n)), seed
    _, _, fl1 = S.rejection_sample(tl, dl, ids, ua, uf, T, 1.0, tk)   # top_p off
    assert not ((fl1 & S.FLAG_TIE_ORDER) != 0).any()
    # an inactive row evaluates no test: only its final draw can flag it
    act = np.zeros(B, bool)
    n3, y3, fl3 = S.rejection_sample(tl, dl, ids, ua, uf, T, tp, tk, active=act)
    assert not n3.any()
    for b in range(B):
        g = S.boundary_tie_group(tl[b, 0], T, tp, tk)
        gq = S.boundary_tie_group(dl[b, 0], T, tp, tk)
        p0 = S.to_probs(tl[b, 0], T, tp, tk)
        q0 = S.to_probs(dl[b, 0], T, tp, tk)
        r = np.maximum(p0 - q0, np.float32(0.0))
        degenerate = rn32(sum(int(v) for v in fixed62(r))) <= np.float32(1e-9)
        in_g = (g is not None and g[y3[b]]) or (not degenerate and gq is not None and gq[y3[b]])
        assert bool(fl3[b] & S.FLAG_TIE_ORDER) == bool(in_g), b

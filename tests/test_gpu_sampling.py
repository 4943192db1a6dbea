"""GPU parity of the HIP sampling path against the oracle (`oracle/sampling.py`).

The kernels are designed to reproduce the oracle bit for bit (same exp rule,
exact fixed-point sums, stable tie order), so probabilities are compared for
exact equality as well as against the 1e-5 absolute tolerance, and every id
/ count / flag is compared exactly.
"""
import numpy as np
import pytest
import torch

from oracle import sampling as O
from specdec import sampling as S
from specdec.workloads import ragged_verify_inputs, uniforms, verify_inputs, zipf_logits

pytestmark = pytest.mark.gpu
DEV = "cuda"

TRANSFORMS = [(1.0, 1.0, 0), (0.8, 0.95, 0), (0.7, 0.9, 50), (1.3, 0.5, 7), (0.6, 0.95, 20),
              (0.0, 1.0, 0)]


def _np(t):
    return t.detach().float().cpu().numpy()


def _assert_probs_equal(got, ref):
    assert got.shape == ref.shape
    assert np.max(np.abs(got - ref)) < 1e-5
    bad = np.nonzero(got.view(np.uint32) != ref.view(np.uint32))
    assert bad[0].size == 0, f"{bad[0].size} elements differ, first at {tuple(b[0] for b in bad)}"


@pytest.mark.parametrize("V,rows", [(64, 16), (1000, 8), (151936, 3)])
@pytest.mark.parametrize("T,tp,tk", TRANSFORMS)
def test_to_probs_bf16(V, rows, T, tp, tk):
    g = torch.Generator(device=DEV).manual_seed(V + rows)
    x = zipf_logits(rows, V, g, DEV)
    got = _np(S.to_probs(x, T, tp, tk))
    ref = O.to_probs(_np(x), T, tp, tk)
    _assert_probs_equal(got, ref)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("T,tp,tk", TRANSFORMS[:4])
def test_to_probs_other_dtypes(dtype, T, tp, tk):
    g = torch.Generator(device=DEV).manual_seed(11)
    x = zipf_logits(6, 4096, g, DEV, dtype=dtype)
    got = _np(S.to_probs(x, T, tp, tk))
    ref = O.to_probs(_np(x), T, tp, tk)
    _assert_probs_equal(got, ref)


def test_to_probs_edge_rows():
    V = 256
    rows = [
        np.zeros(V, np.float32),                                  # one tie group of V
        np.where(np.arange(V) % 3 == 0, 2.0, -1.0).astype(np.float32),
        np.full(V, -np.inf, np.float32),                          # filled below
        np.linspace(-40, 10, V).astype(np.float32),
    ]
    rows[2][[5, 9, 200]] = [1.0, 1.0, 0.5]                        # masked vocab
    x = torch.tensor(np.stack(rows), device=DEV).to(torch.bfloat16)
    for T, tp, tk in [(1.0, 0.3, 0), (0.9, 0.95, 0), (1.0, 1.0, 5), (1.0, 0.5, 100), (2.0, 0.99, 1)]:
        got = _np(S.to_probs(x, T, tp, tk))
        ref = O.to_probs(_np(x), T, tp, tk)
        _assert_probs_equal(got, ref)


def test_to_probs_nonaligned_vocab():
    g = torch.Generator(device=DEV).manual_seed(5)
    x = zipf_logits(4, 1003, g, DEV)
    got = _np(S.to_probs(x, 0.8, 0.9, 0))
    ref = O.to_probs(_np(x), 0.8, 0.9, 0)
    _assert_probs_equal(got, ref)


@pytest.mark.parametrize("B,k,V", [(16, 4, 1000), (4, 4, 151936), (8, 4, 151936), (8, 1, 512),
                                   (6, 8, 4096)])
@pytest.mark.parametrize("T,tp,tk", [(0.8, 0.95, 0), (1.0, 1.0, 0), (0.7, 0.9, 50)])
def test_rejection_sample_bf16(B, k, V, T, tp, tk):
    inp = verify_inputs(B, k, V, seed=B * 100 + k, device=DEV, temperature=T, top_p=tp, top_k=tk)
    n, y, f = S.rejection_sample(inp["target"], inp["draft"], inp["draft_ids"], inp["u_accept"],
                                 inp["u_final"], temperature=T, top_p=tp, top_k=tk)
    rn, ry, rf = O.rejection_sample(_np(inp["target"]), _np(inp["draft"]),
                                    inp["draft_ids"].cpu().numpy(), _np(inp["u_accept"]),
                                    _np(inp["u_final"]), T, tp, tk)
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)


@pytest.mark.parametrize("seed", [1000, 1001])
def test_rejection_sample_bf16_b64_k4_v151936(seed):
    """The full B=64, k=4, V=151936 verify (576 rows: 512 whole, 64 split over
    blocks on a 256-CU device), twice on one workspace."""
    B, k, V, T, tp = 64, 4, 151936, 0.8, 0.95
    inp = verify_inputs(B, k, V, seed=seed, device=DEV, temperature=T, top_p=tp)
    v = S.Verifier(B, k, V, torch.bfloat16, temperature=T, top_p=tp)
    rn, ry, rf = O.rejection_sample(_np(inp["target"]), _np(inp["draft"]),
                                    inp["draft_ids"].cpu().numpy(), _np(inp["u_accept"]),
                                    _np(inp["u_final"]), T, tp, 0)
    for _ in range(2):
        n, y, f = v(inp["target"], inp["draft"], inp["draft_ids"], inp["u_accept"],
                    inp["u_final"])
        assert np.array_equal(n.cpu().numpy(), rn)
        assert np.array_equal(y.cpu().numpy(), ry)
        assert np.array_equal(f.cpu().numpy(), rf)


def test_verifier_graph_replays():
    """The fixed-shape Verifier captured in a graph (nothing in it is a memset:
    counters are cleared by the kernels): replays over two input sets, with
    eager calls and synchronizations between them, each equal to the oracle."""
    B, k, V, T, tp = 16, 4, 151936, 0.8, 0.95
    names = ("target", "draft", "draft_ids", "u_accept", "u_final")
    sets = [verify_inputs(B, k, V, seed=s, device=DEV, temperature=T, top_p=tp) for s in (7, 8)]
    ref = [O.rejection_sample(_np(x["target"]), _np(x["draft"]), x["draft_ids"].cpu().numpy(),
                              _np(x["u_accept"]), _np(x["u_final"]), T, tp, 0) for x in sets]
    v = S.Verifier(B, k, V, torch.bfloat16, temperature=T, top_p=tp)
    static = {n: sets[0][n].clone() for n in names}

    def check(out, i):
        n, y, f = (t.cpu().numpy() for t in out)
        assert np.array_equal(n, ref[i][0])
        assert np.array_equal(y, ref[i][1])
        assert np.array_equal(f, ref[i][2])

    check(v(*(static[n] for n in names)), 0)  # eager, before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = v(*(static[n] for n in names))
    for rep in range(6):
        i = rep % 2
        for n in names:
            static[n].copy_(sets[i][n])
        g.replay()
        torch.cuda.synchronize()
        check(out, i)
        check(v(*(sets[1 - i][n] for n in names)), 1 - i)  # eager work between replays
        torch.cuda.synchronize()


def test_rejection_sample_active_and_fp32():
    B, k, V = 12, 3, 640
    inp = verify_inputs(B, k, V, seed=7, device=DEV, dtype=torch.float32)
    active = torch.tensor([i % 3 != 0 for i in range(B)], device=DEV)
    n, y, f = S.rejection_sample(inp["target"].float(), inp["draft"], inp["draft_ids"],
                                 inp["u_accept"], inp["u_final"], temperature=0.8, top_p=0.95,
                                 active=active)
    rn, ry, rf = O.rejection_sample(_np(inp["target"]), _np(inp["draft"]),
                                    inp["draft_ids"].cpu().numpy(), _np(inp["u_accept"]),
                                    _np(inp["u_final"]), 0.8, 0.95, 0, active.cpu().numpy())
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)
    assert np.all(n.cpu().numpy()[~active.cpu().numpy()] == 0)


def test_rejection_sample_greedy():
    B, k, V = 32, 8, 4096
    g = torch.Generator(device=DEV).manual_seed(3)
    tgt = zipf_logits(B * (k + 1), V, g, DEV).view(B, k + 1, V)
    drf = (tgt[:, :k].float() + torch.randn(B, k, V, generator=g, device=DEV)).to(torch.bfloat16)
    am = tgt[:, :k].float().argmax(-1)
    ids = torch.where(torch.rand(B, k, generator=g, device=DEV) < 0.6, am, (am + 7) % V)
    ua = uniforms((B, k), g, DEV)
    uf = uniforms((B,), g, DEV)
    n, y, f = S.rejection_sample(tgt, drf, ids, ua, uf, temperature=0.0)
    rn, ry, rf = O.rejection_sample(_np(tgt), _np(drf), ids.cpu().numpy(), _np(ua), _np(uf), 0.0)
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)


def test_sample_from_probs_and_residual():
    g = torch.Generator(device=DEV).manual_seed(9)
    V = 3000
    p = S.to_probs(zipf_logits(10, V, g, DEV), 0.9, 0.95)
    q = S.to_probs(zipf_logits(10, V, g, DEV), 0.9, 0.95)
    u = uniforms((10,), g, DEV)
    ids = S.sample_from_probs(p, u=u).cpu().numpy()
    assert np.array_equal(ids, O.sample_from_probs(_np(p), _np(u)))
    r = _np(S.residual_probs(p, q))
    _assert_probs_equal(r, O.residual_probs(_np(p), _np(q)))
    r_deg = _np(S.residual_probs(p, p))                  # degenerate: p itself
    _assert_probs_equal(r_deg, O.residual_probs(_np(p), _np(p)))
    gi = torch.randint(0, V, (10,), generator=g, device=DEV)
    assert np.array_equal(_np(S.gather_prob(p, gi)), O.gather_prob(_np(p), gi.cpu().numpy()))


@pytest.mark.parametrize("V,pad", [(1, 0), (3000, 0), (4096, 0), (4097, 3), (12288, 0),
                                   (12288, 1), (151936, 0), (151936, 5)])
def test_sample_from_probs_records_and_edges(V, pad):
    """Draws over whole 4096-id records, a partial last record and rows whose
    stride is not a multiple of 4 (unaligned, scalar loads), with hand-placed
    rows: all-zero (-1), a single mass at the last id, masses on both sides of
    a record boundary, u = 0 and the largest u below 1, next to random rows."""
    g = torch.Generator(device=DEV).manual_seed(4000 + V + pad)
    rows = 12
    base = torch.zeros(rows, V + pad, device=DEV, dtype=torch.float32)
    p = base[:, :V]
    p[:6] = S.to_probs(zipf_logits(6, V, g, DEV), 0.9, 0.95)
    p[6] = torch.rand(V, generator=g, device=DEV) / V        # dense, unnormalised
    p[7] = 0.0                                                 # all zero
    p[8, V - 1] = 0.25                                         # one mass at the end
    if V > 4096:
        p[9, 4095], p[9, 4096] = 0.5, 0.5                      # across a boundary
    else:
        p[9, 0], p[9, V - 1] = 0.5, 0.5
    p[10] = p[0]
    p[11] = p[1]
    u = uniforms((rows,), g, DEV)
    u[10] = 0.0
    u[11] = float(np.nextafter(np.float32(1.0), np.float32(0.0)))
    if pad:  # straight through the C ABI on the padded rows (stride V + pad)
        from specdec import _lib
        L = _lib.lib()
        out = torch.empty(rows, dtype=torch.int64, device=DEV)
        ws = _lib.workspace(L.sdx_sample_probs_workspace(rows, V), DEV)
        rc = L.sdx_sample_probs(_lib.ptr(base), rows, V, V + pad, _lib.ptr(u), _lib.ptr(out),
                                _lib.ptr(ws), ws.numel(), _lib.stream_of(base))
        _lib.check(rc, "sample_from_probs")
        ids = out.cpu().numpy()
    else:
        ids = S.sample_from_probs(p, u=u).cpu().numpy()
    want = O.sample_from_probs(_np(p), _np(u))
    assert np.array_equal(ids, want), (ids, want)
    assert ids[7] == -1 and ids[8] == V - 1


def test_g1_config1_on_gpu():
    """G1 gate on the HIP path: B=1, k=4, V=64, target N(0, 2^2), draft = target +
    N(0, 0.8^2), T=1, 100,000 trials; first-token TV vs the exact target marginal
    below 0.02, accepted-length histogram vs closed form, and the first 300
    trials bit-exact against the oracle."""
    N, k, V = 100_000, 4, 64
    g = torch.Generator(device=DEV).manual_seed(20241)
    tgt1 = torch.randn(k + 1, V, generator=g, device=DEV) * 2.0
    drf1 = tgt1[:k] + torch.randn(k, V, generator=g, device=DEV) * 0.8
    tgt = tgt1.expand(N, k + 1, V).contiguous()
    drf = drf1.expand(N, k, V).contiguous()
    q = S.to_probs(drf, 1.0)
    ids = S.sample_from_probs(q, u=uniforms((N, k), g, DEV))
    ua, uf = uniforms((N, k), g, DEV), uniforms((N,), g, DEV)
    n, y, _ = S.rejection_sample(tgt, drf, ids, ua, uf, temperature=1.0)
    first = torch.where(n >= 1, ids[:, 0], y).cpu().numpy()
    P = O.to_probs(_np(tgt1), 1.0)
    Q = O.to_probs(_np(drf1), 1.0)
    emp = np.bincount(first, minlength=V) / N
    tv = 0.5 * np.abs(emp - P[0]).sum()
    assert tv < 0.02, tv
    beta = np.minimum(P[:k].astype(np.float64), Q.astype(np.float64)).sum(-1)
    expect = np.array([np.prod(beta[:a]) * (1 - beta[a]) for a in range(k)] + [np.prod(beta)])
    got = np.bincount(n.cpu().numpy(), minlength=k + 1) / N
    assert np.all(np.abs(got - expect) < 5 * np.sqrt(expect * (1 - expect) / N) + 1e-4)
    M = 300
    rn, ry, _ = O.rejection_sample(_np(tgt[:M]), _np(drf[:M]), ids[:M].cpu().numpy(),
                                   _np(ua[:M]), _np(uf[:M]), 1.0)
    assert np.array_equal(n[:M].cpu().numpy(), rn)
    assert np.array_equal(y[:M].cpu().numpy(), ry)


def _window_edge_rows(V):
    """bf16 rows at and beyond the edges of the streaming kernel's fixed value
    window (|x| in [2^-24, 2^16)), which it re-streams into a window anchored
    at the row maximum, mixed with ordinary rows. Rows 0, 2 and 8 hold values
    with |x| >= 2^16."""
    g = np.random.default_rng(17)
    base = (g.standard_normal((10, V)) * 3).astype(np.float32)
    rows = [base[0].copy() for _ in range(10)]
    rows[0][[3, 77]] = [3.0e6, 2.5e6]                     # >= 2^16: leaves the window
    rows[1] = (g.standard_normal(V) * 1e-13).astype(np.float32)   # max among tiny values
    rows[1][[10, 11]] = [0.0, -0.0]
    rows[2][::7] = -3.0e6                                 # <= -2^16: bin 0, zero mass
    rows[3][::5] = 1e-20                                  # tiny values share exp(-m)
    rows[3][1::5] = -1e-30
    rows[4][:] = -np.inf
    rows[4][[1, 2, 3]] = [-1e-14, -2e-14, -2e-14]         # max inside the merged tiny bin
    rows[5] = base[5]                                     # ordinary
    rows[6][::3] = -6.0e4                                 # just inside the window
    rows[7][[0, V - 1]] = [6.5e4, 6.5e4]                  # top of the window, tie at both ends
    rows[8][[5, 6]] = [6.6e4, 6.5e4]                      # 2^16 and just below it
    rows[9][::4] = 7e-8                                   # just above 2^-24
    rows[9][1::4] = -5e-8                                 # just below it
    return np.stack(rows)


@pytest.mark.parametrize("T,tp,tk", [(1.0, 1.0, 0), (0.8, 0.95, 0), (0.7, 0.9, 50),
                                     (3.0e3, 0.9, 0), (4.0e6, 0.9, 0), (4.0e6, 1.0, 0)])
def test_to_probs_bf16_window_edges(T, tp, tk):
    V = 4096
    x = torch.tensor(_window_edge_rows(V), device=DEV).to(torch.bfloat16)
    got = _np(S.to_probs(x, T, tp, tk))
    ref = O.to_probs(_np(x), T, tp, tk)
    # rows the kernels cannot represent come back as NaN (the C API also flags
    # them in verify); only absurd temperatures on rows with |x| >= 2^16 produce them
    bad = np.isnan(got).any(axis=1)
    assert not np.isnan(got[~bad]).any()
    if T < 1e3:
        assert not bad.any()
    assert set(np.flatnonzero(bad)) <= {0, 2, 8}
    _assert_probs_equal(got[~bad], ref[~bad])


def test_rejection_sample_window_edges_and_nonfinite():
    B, k, V = 4, 1, 4096
    rows = _window_edge_rows(V)[:8]
    tgt = torch.tensor(rows, device=DEV).to(torch.bfloat16).view(B, 2, V)
    drf = torch.tensor(rows[::-1].copy(), device=DEV).to(torch.bfloat16)[:B].view(B, 1, V)
    g = torch.Generator(device=DEV).manual_seed(4)
    ids = torch.tensor([[3], [10], [0], [1]], device=DEV)
    ua, uf = uniforms((B, k), g, DEV), uniforms((B,), g, DEV)
    for T, tp in [(1.0, 1.0), (0.8, 0.95)]:
        n, y, f = S.rejection_sample(tgt, drf, ids, ua, uf, temperature=T, top_p=tp)
        rn, ry, rf = O.rejection_sample(_np(tgt), _np(drf), ids.cpu().numpy(), _np(ua), _np(uf),
                                        T, tp, 0)
        fin = (rf & 2) == 0                    # rows with +inf/NaN are unspecified
        assert np.array_equal(f.cpu().numpy() & 2, rf & 2)
        assert np.array_equal(n.cpu().numpy()[fin], rn[fin])
        assert np.array_equal(y.cpu().numpy()[fin], ry[fin])
    bad = tgt.clone()
    bad[1, 0, 9] = float("inf")
    _, _, f = S.rejection_sample(bad, drf, ids, ua, uf, temperature=1.0)
    assert int(f[1]) & 2


def _tie_heavy(shape, g, step=0.5, sigma=2.0):
    """Logits on a coarse grid: boundary tie groups of thousands of members
    spanning many id chunks."""
    x = torch.randn(shape, generator=g, device=DEV) * sigma
    return (torch.round(x / step) * step).to(torch.bfloat16)


@pytest.mark.parametrize("T,tp,tk", [(1.0, 0.9, 0), (0.8, 0.5, 0), (1.0, 0.97, 3000)])
def test_to_probs_bf16_large_tie_groups(T, tp, tk):
    g = torch.Generator(device=DEV).manual_seed(31)
    x = _tie_heavy((4, 151936), g)
    got = _np(S.to_probs(x, T, tp, tk))
    ref = O.to_probs(_np(x), T, tp, tk)
    _assert_probs_equal(got, ref)


@pytest.mark.parametrize("T,tp", [(1.0, 0.9), (0.8, 0.6)])
def test_rejection_sample_large_tie_groups(T, tp):
    """Draft tokens drawn from inside the target's boundary tie group (some
    kept, some dropped by id order), residual draws across group chunks."""
    B, k, V = 6, 3, 151936
    g = torch.Generator(device=DEV).manual_seed(41)
    tgt = _tie_heavy((B, k + 1, V), g)
    drf = _tie_heavy((B, k, V), g, sigma=2.2)
    P = O.to_probs(_np(tgt[:, :k]).reshape(B * k, V), T, tp, 0)
    xt = _np(tgt[:, :k]).reshape(B * k, V)
    rng = np.random.default_rng(5)
    ids = np.empty(B * k, np.int64)
    for r in range(B * k):
        vmin = xt[r][P[r] > 0].min()              # boundary value of the nucleus
        grp = np.nonzero(xt[r] == vmin)[0]
        ids[r] = grp[rng.integers(len(grp))]
    ids = torch.tensor(ids.reshape(B, k), device=DEV)
    ua = uniforms((B, k), g, DEV) * 0.05             # mostly accept: exercise later positions
    ua[::2] = uniforms((B // 2, k), g, DEV)
    uf = uniforms((B,), g, DEV)
    n, y, f = S.rejection_sample(tgt, drf, ids, ua, uf, temperature=T, top_p=tp)
    rn, ry, rf = O.rejection_sample(_np(tgt), _np(drf), ids.cpu().numpy(), _np(ua), _np(uf),
                                    T, tp, 0)
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)


def _tiny_tie_rows(n, V, rng):
    """Rows of ten logits 3.0 and the rest tiny values (|x| < 2^-24, many bf16
    codes) that share one probability: one boundary tie group of many values."""
    x = (rng.standard_normal((n, V)) * 1e-9).astype(np.float32)
    x[:, ::7] = 0.0
    x[:, 1::11] = -0.0
    x[:, :10] = 3.0
    return x


@pytest.mark.parametrize("T,tp", [(1.0, 0.5), (1.0, 0.8)])
def test_rejection_sample_multivalue_tie_group_ranks(T, tp):
    """Drafted tokens inside a partial boundary tie group spanning many values
    (the merged tiny-value bin): their member ranks come from the accept chain."""
    B, k, V = 4, 2, 4096
    rng = np.random.default_rng(9)
    tgt_np = _tiny_tie_rows(B * (k + 1), V, rng).reshape(B, k + 1, V)
    drf_np = _tiny_tie_rows(B * k, V, rng).reshape(B, k, V)
    tgt = torch.tensor(tgt_np, device=DEV).to(torch.bfloat16)
    drf = torch.tensor(drf_np, device=DEV).to(torch.bfloat16)
    ids = torch.tensor(rng.integers(10, V, (B, k)), device=DEV)
    g = torch.Generator(device=DEV).manual_seed(12)
    ua = uniforms((B, k), g, DEV) * 0.5
    uf = uniforms((B,), g, DEV)
    n, y, f = S.rejection_sample(tgt, drf, ids, ua, uf, temperature=T, top_p=tp)
    rn, ry, rf = O.rejection_sample(_np(tgt), _np(drf), ids.cpu().numpy(), _np(ua), _np(uf),
                                    T, tp, 0)
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)


# ---------------------------------------------------------------- per-row k
def _ragged_oracle(inp, T, tp, tk, active=None):
    return O.rejection_sample_ragged(_np(inp["target"]), _np(inp["draft"]),
                                     inp["draft_ids"].cpu().numpy(), _np(inp["u_accept"]),
                                     _np(inp["u_final"]), inp["cu_k"].cpu().numpy(), T, tp, tk,
                                     active)


@pytest.mark.parametrize("T,tp,tk", [(0.7, 0.9, 50), (0.8, 0.95, 0), (0.0, 1.0, 0)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rejection_sample_ragged_matches_oracle(T, tp, tk, dtype):
    """Rows of k_b from 0 to 8 packed in one call (k_b = 0: bonus draw only)."""
    ks = [3, 0, 8, 1, 5, 2, 8, 4, 0, 6]
    inp = ragged_verify_inputs(len(ks), 4096, seed=21, device=DEV, temperature=T, top_p=tp,
                               top_k=tk, dtype=dtype, k=ks)
    n, y, f = S.rejection_sample_ragged(inp["target"], inp["draft"], inp["draft_ids"],
                                        inp["u_accept"], inp["u_final"], inp["cu_k"], k_max=8,
                                        temperature=T, top_p=tp, top_k=tk)
    rn, ry, rf = _ragged_oracle(inp, T, tp, tk)
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)


def test_rejection_sample_ragged_config5_vocab():
    """Config 5's sampler: k_b from the controller at alpha_b ~ U(0.4, 0.9),
    c = 0.1, V = 151936 bf16, T = 0.7, top-k 50, top-p 0.9; some rows inactive."""
    B = 24
    inp = ragged_verify_inputs(B, 151936, seed=5, device=DEV)
    active = torch.tensor([b % 5 != 2 for b in range(B)], device=DEV)
    n, y, f = S.rejection_sample_ragged(inp["target"], inp["draft"], inp["draft_ids"],
                                        inp["u_accept"], inp["u_final"], inp["cu_k"],
                                        temperature=0.7, top_p=0.9, top_k=50, active=active)
    rn, ry, rf = _ragged_oracle(inp, 0.7, 0.9, 50, active.cpu().numpy())
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)


def test_rejection_sample_ragged_graph_replays():
    """Per-row k captured in a graph (k_max, workspace and outputs given, so the
    call makes no host sync): replays over two input sets of one row layout,
    with eager calls between, each equal to the oracle."""
    from specdec import _lib
    B, V = 16, 151936
    ks = [1 + (3 * b) % 8 for b in range(B)]
    names = ("target", "draft", "draft_ids", "u_accept", "u_final", "cu_k")
    sets = [ragged_verify_inputs(B, V, seed=s, device=DEV, k=ks) for s in (11, 12)]
    ref = [_ragged_oracle(x, 0.7, 0.9, 50) for x in sets]
    static = {n: sets[0][n].clone() for n in names}
    ws = _lib.workspace(_lib.lib().sdx_verify_ragged_workspace(B, sum(ks) + B, V, _lib.BF16), DEV)
    out = (torch.empty(B, dtype=torch.int64, device=DEV),
           torch.empty(B, dtype=torch.int64, device=DEV),
           torch.empty(B, dtype=torch.uint8, device=DEV))

    def call(src):
        return S.rejection_sample_ragged(src["target"], src["draft"], src["draft_ids"],
                                         src["u_accept"], src["u_final"], src["cu_k"],
                                         k_max=max(ks), temperature=0.7, top_p=0.9, top_k=50,
                                         workspace=ws, out=out)

    def check(res, i):
        for got, want in zip(res, ref[i]):
            assert np.array_equal(got.cpu().numpy(), want)

    check(call(static), 0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        res = call(static)
    for rep in range(6):
        i = rep % 2
        for n in names:
            static[n].copy_(sets[i][n])
        g.replay()
        torch.cuda.synchronize()
        check(res, i)
        check(call(sets[1 - i]), 1 - i)  # eager work between replays
        torch.cuda.synchronize()


def test_rejection_sample_ragged_equal_k_is_uniform():
    """cu_k = 4 * arange(B+1) over the reshaped B=64, k=4, V=151936 step gives
    the uniform verify bit for bit (576 rows, split rows included)."""
    B, k, V, T, tp = 64, 4, 151936, 0.8, 0.95
    inp = verify_inputs(B, k, V, seed=1000, device=DEV, temperature=T, top_p=tp)
    n, y, f = S.rejection_sample(inp["target"], inp["draft"], inp["draft_ids"], inp["u_accept"],
                                 inp["u_final"], temperature=T, top_p=tp)
    cu = torch.arange(B + 1, device=DEV, dtype=torch.int64) * k
    n2, y2, f2 = S.rejection_sample_ragged(inp["target"].reshape(-1, V), inp["draft"].reshape(-1, V),
                                           inp["draft_ids"].reshape(-1),
                                           inp["u_accept"].reshape(-1), inp["u_final"], cu,
                                           k_max=k, temperature=T, top_p=tp)
    assert torch.equal(n, n2) and torch.equal(y, y2) and torch.equal(f, f2)


def test_rejection_sample_ragged_rejects_bad_offsets():
    """Offsets that decrease, or a k_b above k_max, flag every row and accept nothing."""
    ks = [2, 3, 1]
    inp = ragged_verify_inputs(3, 512, seed=3, device=DEV, k=ks)
    for cu in ([0, 4, 3, 6], [0, 2, 5, 6]):
        cu_k = torch.tensor(cu, dtype=torch.int64, device=DEV)
        kmax = 2 if cu == [0, 2, 5, 6] else 8   # second: k_1 = 3 > k_max = 2
        n, y, f = S.rejection_sample_ragged(inp["target"], inp["draft"], inp["draft_ids"],
                                            inp["u_accept"], inp["u_final"], cu_k, k_max=kmax,
                                            temperature=0.7, top_p=0.9, top_k=50)
        assert np.all(f.cpu().numpy() & S.FLAG_BAD_ROW)
        assert np.all(n.cpu().numpy() == 0)


@pytest.mark.parametrize("seed", range(4))
def test_rejection_sample_ragged_random(seed):
    """Seeded random row counts, k lists (0 to k_max), vocab and transform."""
    rng = np.random.RandomState(seed)
    B = int(rng.randint(1, 20))
    k_max = int(rng.randint(1, 12))
    ks = [int(x) for x in rng.randint(0, k_max + 1, B)]
    V = int(rng.choice([64, 1000, 4096]))
    T, tp, tk = [(0.7, 0.9, 50), (1.0, 1.0, 0), (1.3, 0.5, 7), (0.0, 1.0, 0)][seed]
    inp = ragged_verify_inputs(B, V, seed=seed + 50, device=DEV, temperature=T, top_p=tp,
                               top_k=tk, k=ks)
    n, y, f = S.rejection_sample_ragged(inp["target"], inp["draft"], inp["draft_ids"],
                                        inp["u_accept"], inp["u_final"], inp["cu_k"],
                                        k_max=k_max, temperature=T, top_p=tp, top_k=tk)
    rn, ry, rf = _ragged_oracle(inp, T, tp, tk)
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)


def _coarse_logits(shape, g, dtype):
    """Logits on a grid of 0.5 (12 values): every probability is shared by many
    tokens, so a top-p cut nearly always falls inside a tie group."""
    x = torch.randint(0, 12, shape, generator=g, device=DEV).float() * 0.5 - 3.0
    return x.to(dtype)


def _ids_in_groups(drf, T, tp, tk, g):
    """Draft ids: a member of the draft row's partially kept boundary group with
    probability 0.7, else any id."""
    d = _np(drf)
    sh = d.shape[:-1]
    V = d.shape[-1]
    pick = torch.rand(sh, generator=g, device=DEV).cpu().numpy()
    anyid = torch.randint(0, V, sh, generator=g, device=DEV).cpu().numpy()
    out = np.zeros(sh, np.int64)
    for idx in np.ndindex(*sh):
        grp = O.boundary_tie_group(d[idx], T, tp, tk)
        if grp is not None and pick[idx] < 0.7:
            mem = np.flatnonzero(grp)
            out[idx] = mem[int(anyid[idx]) % mem.size]
        else:
            out[idx] = anyid[idx]
    return torch.from_numpy(out).to(DEV)


@pytest.mark.parametrize("dtype,V,k", [(torch.bfloat16, 4096, 4), (torch.float16, 4096, 4),
                                       (torch.float32, 2048, 3), (torch.bfloat16, 151936, 4),
                                       (torch.bfloat16, 1024, 40)])
def test_tie_order_flags(dtype, V, k):
    """SDX_FLAG_TIE_ORDER (32) on rows whose accept tests or final draw touch a
    partially kept top-p boundary tie group: flags equal the oracle's, bit for
    bit, with accept-side and draw-side cases both present."""
    B, T, tp, tk = 16, 0.9, 0.8, 0
    g = torch.Generator(device=DEV).manual_seed(V + k)
    tgt = _coarse_logits((B, k + 1, V), g, dtype)
    drf = (tgt[:, :k].float() + 0.5 * torch.randint(0, 2, (B, k, V), generator=g,
                                                     device=DEV).float()).to(dtype)
    ids = _ids_in_groups(drf, T, tp, tk, g)
    ua = uniforms((B, k), g, DEV)
    uf = uniforms((B,), g, DEV)
    n, y, f = S.rejection_sample(tgt, drf, ids, ua, uf, temperature=T, top_p=tp, top_k=tk)
    rn, ry, rf = O.rejection_sample(_np(tgt), _np(drf), ids.cpu().numpy(), _np(ua), _np(uf),
                                    T, tp, tk)
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)
    tied = (rf & O.FLAG_TIE_ORDER) != 0
    assert tied.any() and not tied.all()
    # with top_p off nothing is flagged
    n, y, f = S.rejection_sample(tgt, drf, ids, ua, uf, temperature=T, top_p=1.0, top_k=tk)
    assert not (f.cpu().numpy() & O.FLAG_TIE_ORDER).any()


def test_tie_order_flags_ragged():
    """The flag through the per-row-k verify (rows with k_b = 0 included)."""
    B, V, T, tp = 12, 4096, 0.9, 0.8
    g = torch.Generator(device=DEV).manual_seed(77)
    kb = torch.randint(0, 6, (B,), generator=g, device=DEV).cpu().numpy()
    cu = np.concatenate([[0], np.cumsum(kb)]).astype(np.int64)
    nt = int(cu[-1]) + B
    tgt = _coarse_logits((nt, V), g, torch.bfloat16)
    tidx = np.concatenate([np.arange(cu[b] + b, cu[b] + b + kb[b]) for b in range(B)])
    drf = (tgt[torch.from_numpy(tidx).to(DEV)].float() + 0.5 * torch.randint(
        0, 2, (int(cu[-1]), V), generator=g, device=DEV).float()).to(torch.bfloat16)
    ids = _ids_in_groups(drf, T, tp, 0, g)
    ua = uniforms((int(cu[-1]),), g, DEV)
    uf = uniforms((B,), g, DEV)
    cu_t = torch.from_numpy(cu).to(DEV)
    n, y, f = S.rejection_sample_ragged(tgt, drf, ids, ua, uf, cu_t, temperature=T, top_p=tp)
    rn, ry, rf = O.rejection_sample_ragged(_np(tgt), _np(drf), ids.cpu().numpy(), _np(ua),
                                           _np(uf), cu, T, tp, 0)
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)
    assert ((rf & O.FLAG_TIE_ORDER) != 0).any()

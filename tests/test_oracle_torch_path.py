"""Pins of the torch CPU restatement that bench.py times as its CPU baseline
(`oracle/torch_path.py`) against the numpy oracle: same transform to
rounding, same accept decisions away from near-ties, same draws."""
import numpy as np
import torch

from oracle import sampling as O
from oracle import torch_path as TP


def _inputs(B, k, V, seed):
    g = torch.Generator().manual_seed(seed)
    tgt = (torch.randn(B, k + 1, V, generator=g) * 3).to(torch.bfloat16)
    drf = (tgt[:, :k].float() + torch.randn(B, k, V, generator=g)).to(torch.bfloat16)
    q = TP.to_probs(drf, 0.8, 0.95)
    ids = torch.multinomial(q.reshape(-1, V), 1, generator=g).view(B, k)
    ua = torch.rand(B, k, generator=g)
    uf = torch.rand(B, generator=g)
    return tgt, drf, ids, ua, uf


def test_to_probs_matches_oracle():
    tgt, _, _, _, _ = _inputs(4, 2, 4096, 1)
    x = tgt.reshape(-1, 4096)
    for T, tp, tk in [(0.8, 0.95, 0), (0.7, 0.9, 50), (1.0, 1.0, 0), (0.0, 1.0, 0)]:
        got = TP.to_probs(x, T, tp, tk).numpy()
        ref = O.to_probs(x.float().numpy(), T, tp, tk)
        assert np.max(np.abs(got - ref)) < 1e-5


def test_rejection_sample_matches_oracle():
    B, k, V = 32, 4, 4096
    tgt, drf, ids, ua, uf = _inputs(B, k, V, 7)
    n, y = TP.rejection_sample(tgt, drf, ids, ua, uf, 0.8, 0.95, 0)
    rn, ry, rf = O.rejection_sample(tgt.float().numpy(), drf.float().numpy(), ids.numpy(),
                                    ua.numpy(), uf.numpy(), 0.8, 0.95, 0)
    calm = (rf & O.FLAG_ACCEPT_NEAR_TIE) == 0
    assert np.array_equal(n.numpy()[calm], rn[calm])
    assert 0 < rn.sum() < B * k                       # accepts and rejects both occur
    assert (y.numpy() == ry).mean() >= 0.95           # draws agree away from rounding edges


def test_greedy_matches_oracle():
    B, k, V = 16, 3, 1000
    tgt, drf, ids, ua, uf = _inputs(B, k, V, 9)
    am = tgt[:, :k].float().argmax(-1)
    ids = torch.where(torch.arange(B * k).view(B, k) % 3 == 0, (am + 1) % V, am)
    n, y = TP.rejection_sample(tgt, drf, ids, ua, uf, 0.0)
    rn, ry, _ = O.greedy_verify(tgt.float().numpy(), ids.numpy(), ua.numpy())
    assert np.array_equal(n.numpy(), rn) and np.array_equal(y.numpy(), ry)

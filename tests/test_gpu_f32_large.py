"""fp32 logits above 8,192 tokens (the multi-pass kernel that sorts only the
nucleus boundary region) against the oracle, bit for bit: to_probs over the
transforms of the other parity tests, rows of heavy ties (coarse logits: tie
groups of equal values) and of equal probabilities from distinct values
(logits so close that exp rounds them together, so a tie group spans several
keys), the verify at Qwen3's vocabulary with the tie-order flag, and the vocab
limit."""
import numpy as np
import pytest
import torch

from oracle import sampling as O
from specdec import sampling as S
from specdec.workloads import uniforms, verify_inputs, zipf_logits

pytestmark = pytest.mark.gpu
DEV = "cuda"
TRANSFORMS = [(1.0, 1.0, 0), (0.8, 0.95, 0), (0.7, 0.9, 50), (1.3, 0.5, 7), (0.6, 0.95, 20),
              (0.0, 1.0, 0), (1.0, 0.99, 2000)]


def _np(t):
    return t.detach().float().cpu().numpy()


def _assert_probs_equal(got, ref):
    assert got.shape == ref.shape
    assert np.max(np.abs(got - ref)) < 1e-5
    bad = np.nonzero(got.view(np.uint32) != ref.view(np.uint32))
    assert bad[0].size == 0, f"{bad[0].size} elements differ, first at {tuple(b[0] for b in bad)}"


# 8203: output rows that do not start 16-byte aligned (the kernel's one-id-per-thread
# output path) next to aligned ones
@pytest.mark.parametrize("V", [8200, 8203, 151936])
@pytest.mark.parametrize("T,tp,tk", TRANSFORMS)
def test_to_probs_f32_large(V, T, tp, tk):
    print(f"[f32] V={V} T={T} tp={tp} tk={tk}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(V + int(100 * T) + tk)
    x = zipf_logits(3, V, g, DEV, dtype=torch.float32)
    _assert_probs_equal(_np(S.to_probs(x, T, tp, tk)), O.to_probs(_np(x), T, tp, tk))


@pytest.mark.parametrize("T,tp,tk", [(1.0, 0.9, 0), (0.9, 0.7, 0), (1.0, 0.95, 300), (1.0, 0.3, 0)])
def test_to_probs_f32_large_ties(T, tp, tk):
    V = 151936
    rng = np.random.default_rng(int(10 * T) + tk)
    rows = [
        np.round(rng.standard_normal(V) * 4) / 4,                 # tie groups of equal values
        np.round(rng.standard_normal(V) * 2),                     # few, huge tie groups
        rng.standard_normal(V) * 1e-6,                            # equal p from distinct values
        np.linspace(-3, 3, V),
    ]
    x = torch.tensor(np.stack(rows).astype(np.float32), device=DEV)
    _assert_probs_equal(_np(S.to_probs(x, T, tp, tk)), O.to_probs(_np(x), T, tp, tk))


@pytest.mark.parametrize("T,tp,tk", [(0.8, 0.95, 0), (0.7, 0.9, 50), (1.0, 1.0, 0)])
def test_rejection_sample_f32_qwen3_vocab(T, tp, tk):
    B, k, V = 4, 4, 151936
    inp = verify_inputs(B, k, V, seed=31 + tk, device=DEV, temperature=T, top_p=tp, top_k=tk,
                        dtype=torch.float32)
    n, y, f = S.rejection_sample(inp["target"], inp["draft"], inp["draft_ids"], inp["u_accept"],
                                 inp["u_final"], temperature=T, top_p=tp, top_k=tk)
    rn, ry, rf = O.rejection_sample(_np(inp["target"]), _np(inp["draft"]),
                                    inp["draft_ids"].cpu().numpy(), _np(inp["u_accept"]),
                                    _np(inp["u_final"]), T, tp, tk)
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)


def test_rejection_sample_f32_tie_groups():
    """Coarse fp32 logits: drafted tokens and draws inside partially kept tie
    groups; n_acc, y and flags (the tie-order bit included) as the oracle."""
    B, k, V, T, tp = 8, 3, 20000, 0.9, 0.8
    rng = np.random.default_rng(5)
    tgt = np.round(rng.standard_normal((B, k + 1, V)) * 2) / 2
    drf = tgt[:, :k] + 0.5 * rng.integers(0, 2, (B, k, V))
    tgt_t = torch.tensor(tgt.astype(np.float32), device=DEV)
    drf_t = torch.tensor(drf.astype(np.float32), device=DEV)
    g = torch.Generator(device=DEV).manual_seed(2)
    q = S.to_probs(drf_t, T, tp, 0)
    ids = S.sample_from_probs(q, u=uniforms((B, k), g, DEV))
    ua, uf = uniforms((B, k), g, DEV), uniforms((B,), g, DEV)
    n, y, f = S.rejection_sample(tgt_t, drf_t, ids, ua, uf, temperature=T, top_p=tp)
    rn, ry, rf = O.rejection_sample(tgt.astype(np.float32), drf.astype(np.float32),
                                    ids.cpu().numpy(), _np(ua), _np(uf), T, tp, 0)
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)
    assert ((rf & O.FLAG_TIE_ORDER) != 0).any()


def test_f32_vocab_limit():
    g = torch.Generator(device=DEV).manual_seed(3)
    with pytest.raises(RuntimeError, match="vocab"):
        S.to_probs(zipf_logits(1, 262144 + 8, g, DEV, dtype=torch.float32), 0.8, 0.95, 0)

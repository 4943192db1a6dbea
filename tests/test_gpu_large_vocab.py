"""GPU parity at vocabularies above 163,840 (bf16 logits up to 262,136): the
sizes of 200K-vocabulary models (202,048) and the largest bf16 row the row
kernel takes (2^18 - 8, every per-bin count below 2^18). Same bar as the other
sampling tests: probabilities bit-identical to the oracle, ids / counts / flags
exact. fp16 rows above 163,840 (the fp16 kernels' limit: their row kernel
holds a row in registers) are widened to fp32 by the Python entry points and
run on the fp32 kernels: the same bar, through every entry point.
"""
import numpy as np
import pytest
import torch

from oracle import sampling as O
from specdec import sampling as S
from specdec.workloads import ragged_verify_inputs, uniforms, verify_inputs, zipf_logits

pytestmark = pytest.mark.gpu
DEV = "cuda"
V_MAX_BF16 = (1 << 18) - 8


def _np(t):
    return t.detach().float().cpu().numpy()


def _assert_probs_equal(got, ref):
    assert got.shape == ref.shape
    assert np.max(np.abs(got - ref)) < 1e-5
    bad = np.nonzero(got.view(np.uint32) != ref.view(np.uint32))
    assert bad[0].size == 0, f"{bad[0].size} elements differ, first at {tuple(b[0] for b in bad)}"


@pytest.mark.parametrize("V", [202048, V_MAX_BF16])
@pytest.mark.parametrize("T,tp,tk", [(0.8, 0.95, 0), (0.7, 0.9, 50), (0.0, 1.0, 0)])
def test_to_probs_bf16_large_vocab(V, T, tp, tk):
    g = torch.Generator(device=DEV).manual_seed(V + int(100 * tp))
    x = zipf_logits(3, V, g, DEV)
    _assert_probs_equal(_np(S.to_probs(x, T, tp, tk)), O.to_probs(_np(x), T, tp, tk))


def test_to_probs_bf16_large_vocab_one_tie_group():
    """Every logit equal: one tie group of V members (the largest count a bin holds)."""
    x = torch.zeros((2, V_MAX_BF16), dtype=torch.bfloat16, device=DEV)
    x[1, ::3] = 1.0
    for T, tp in ((1.0, 1.0), (0.8, 0.5)):
        _assert_probs_equal(_np(S.to_probs(x, T, tp, 0)), O.to_probs(_np(x), T, tp, 0))


@pytest.mark.parametrize("V,B,k", [(202048, 8, 4), (V_MAX_BF16, 6, 3)])
def test_rejection_sample_bf16_large_vocab(V, B, k):
    T, tp = 0.8, 0.95
    inp = verify_inputs(B, k, V, seed=V + B, device=DEV, temperature=T, top_p=tp)
    rn, ry, rf = O.rejection_sample(_np(inp["target"]), _np(inp["draft"]),
                                    inp["draft_ids"].cpu().numpy(), _np(inp["u_accept"]),
                                    _np(inp["u_final"]), T, tp, 0)
    for _ in range(2):  # twice on the library's cached workspace
        n, y, f = S.rejection_sample(inp["target"], inp["draft"], inp["draft_ids"],
                                     inp["u_accept"], inp["u_final"], temperature=T, top_p=tp)
        assert np.array_equal(n.cpu().numpy(), rn)
        assert np.array_equal(y.cpu().numpy(), ry)
        assert np.array_equal(f.cpu().numpy(), rf)


def test_rejection_sample_ragged_bf16_large_vocab():
    T, tp, tk = 0.7, 0.9, 50
    ks = [0, 3, 8, 1, 5, 2]
    inp = ragged_verify_inputs(len(ks), V_MAX_BF16, seed=41, device=DEV, temperature=T,
                               top_p=tp, top_k=tk, k=ks)
    n, y, f = S.rejection_sample_ragged(inp["target"], inp["draft"], inp["draft_ids"],
                                        inp["u_accept"], inp["u_final"], inp["cu_k"],
                                        temperature=T, top_p=tp, top_k=tk)
    rn, ry, rf = O.rejection_sample_ragged(_np(inp["target"]), _np(inp["draft"]),
                                           inp["draft_ids"].cpu().numpy(), _np(inp["u_accept"]),
                                           _np(inp["u_final"]), inp["cu_k"].cpu().numpy(), T, tp,
                                           tk)
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)


def test_greedy_verify_large_vocab():
    B, k, V = 4, 4, V_MAX_BF16
    g = torch.Generator(device=DEV).manual_seed(5)
    tgt = zipf_logits(B * (k + 1), V, g, DEV).view(B, k + 1, V)
    flat = tgt.view(-1, V)
    flat[0, V - 1] = flat[0].float().max() + 1.0  # the maximum at the last id
    flat[1, 7] = flat[1, V - 8] = flat[1].float().max() + 1.0  # tied maxima: the first wins
    am = flat.float().argmax(dim=1).view(B, k + 1)
    ids = am[:, :k].clone()
    ids[1, 2] = (ids[1, 2] + 1) % V
    ids[3, 0] = (ids[3, 0] + 5) % V
    ua = uniforms((B, k), g, DEV)
    uf = torch.zeros(B, dtype=torch.float32, device=DEV)
    n, y, f = S.rejection_sample(tgt, None, ids, ua, uf, temperature=0.0)
    rn, ry, rf = O.greedy_verify(_np(tgt), ids.cpu().numpy(), _np(ua))
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)


def test_sample_from_probs_large_vocab():
    g = torch.Generator(device=DEV).manual_seed(9)
    p = S.to_probs(zipf_logits(4, V_MAX_BF16, g, DEV), 0.8, 0.95, 0)
    u = uniforms((4,), g, DEV)
    got = S.sample_from_probs(p, u=u).cpu().numpy()
    assert np.array_equal(got, O.sample_from_probs(_np(p), _np(u)))


def test_vocab_limits_by_dtype():
    """Above the limits the library refuses the shape (SDX_EUNSUPPORTED) before
    any launch: bf16 past 2^18 - 8. fp16 past 163,840 is refused by the C ABI
    (tests/test_boundary.py) and served by the Python entry points through the
    fp32 kernels."""
    g = torch.Generator(device=DEV).manual_seed(3)
    with pytest.raises(RuntimeError, match="vocab"):
        S.to_probs(zipf_logits(1, V_MAX_BF16 + 8, g, DEV), 0.8, 0.95, 0)
    for dt in (torch.bfloat16, torch.float16):  # both served at that size
        x = zipf_logits(1, 163840 + 8, g, DEV, dtype=dt)
        _assert_probs_equal(_np(S.to_probs(x, 0.8, 0.95, 0)), O.to_probs(_np(x), 0.8, 0.95, 0))


@pytest.mark.parametrize("V", [163848, 202048])
def test_fp16_rows_above_the_fp16_kernels(V):
    """fp16 rows longer than the fp16 kernels take, through to_probs,
    draft_step, rejection_sample, rejection_sample_ragged and the prepared
    Verifier (its fp32 copies), against the oracle on the same fp16 values."""
    T, tp, B, k = 0.8, 0.95, 4, 3
    g = torch.Generator(device=DEV).manual_seed(V)
    x = zipf_logits(3, V, g, DEV, dtype=torch.float16)
    _assert_probs_equal(_np(S.to_probs(x, T, tp, 0)), O.to_probs(_np(x), T, tp, 0))
    u = uniforms((3,), g, DEV)
    xd, qx, _ = S.draft_step(x, u, T, tp)
    rx = O.sample_from_probs(O.to_probs(_np(x), T, tp, 0), _np(u))
    assert np.array_equal(xd.cpu().numpy(), rx)
    inp = verify_inputs(B, k, V, seed=V + 1, device=DEV, temperature=T, top_p=tp,
                        dtype=torch.float16)
    args = (inp["target"], inp["draft"], inp["draft_ids"], inp["u_accept"], inp["u_final"])
    rn, ry, rf = O.rejection_sample(_np(inp["target"]), _np(inp["draft"]),
                                    inp["draft_ids"].cpu().numpy(), _np(inp["u_accept"]),
                                    _np(inp["u_final"]), T, tp, 0)
    outs = [S.rejection_sample(*args, temperature=T, top_p=tp)]
    ver = S.Verifier(B, k, V, torch.float16, temperature=T, top_p=tp, device=DEV)
    outs.append(ver(*args))
    cu = torch.arange(0, B * k + 1, k, dtype=torch.int64, device=DEV)
    tl = inp["target"].reshape(B * (k + 1), V)
    dl = inp["draft"].reshape(B * k, V)
    outs.append(S.rejection_sample_ragged(tl, dl, inp["draft_ids"].reshape(-1),
                                          inp["u_accept"].reshape(-1), inp["u_final"], cu,
                                          k_max=k, temperature=T, top_p=tp))
    for n, y, f in outs:
        assert np.array_equal(n.cpu().numpy(), rn)
        assert np.array_equal(y.cpu().numpy(), ry)
        assert np.array_equal(f.cpu().numpy(), rf)

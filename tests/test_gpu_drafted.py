"""`sdx_verify_drafted` (`Verifier.drafted`): the verify of a round whose draft
rows went through `draft_step`, taking their statistics from the draft steps'
workspaces instead of streaming the draft logits again. It must equal the
plain verify (and the oracle) bit for bit: n_acc, y and flags, for drafted ids
drawn by the draft steps and for any other ids (whose probabilities, tie-group
ranks included, are then set from the gathered statistics). Draft workspaces
made at another sampling configuration flag every row SDX_FLAG_WORKSPACE."""
import numpy as np
import pytest
import torch

from oracle import sampling as O
from specdec import _lib
from specdec.sampling import FLAG_WORKSPACE, Verifier, draft_step
from specdec.workloads import uniforms, verify_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().float().cpu().numpy()


def _draft_steps(draft, T, tp, tk, seed, k, B, V):
    """k draft steps on draft[:, i]: ids [B, k] and the k workspaces."""
    L = _lib.lib()
    g = torch.Generator(device=DEV).manual_seed(seed)
    wss = [_lib.workspace(L.sdx_draft_step_workspace(B, V, _lib.BF16), DEV) for _ in range(k)]
    xs = []
    for i in range(k):
        x, _, _ = draft_step(draft[:, i], uniforms((B,), g, DEV), T, tp, tk, workspace=wss[i])
        xs.append(x.clone())
    return torch.stack(xs, 1).contiguous(), wss


@pytest.mark.parametrize("B,k,V,T,tp,tk", [(64, 4, 151936, 0.8, 0.95, 0),
                                           (16, 3, 32000, 0.7, 0.9, 50),
                                           (9, 8, 4096, 1.0, 1.0, 0),
                                           (5, 2, 151936, 0.6, 0.5, 0)])
def test_drafted_equals_plain_verify(B, k, V, T, tp, tk):
    print(f"[drafted] B={B} k={k} V={V} T={T} tp={tp} tk={tk}", flush=True)
    inp = verify_inputs(B, k, V, seed=400 + V % 97 + k, device=DEV, temperature=T, top_p=tp,
                        top_k=tk)
    ids, wss = _draft_steps(inp["draft"], T, tp, tk, 17 + B, k, B, V)
    v = Verifier(B, k, V, torch.bfloat16, temperature=T, top_p=tp, top_k=tk, device=DEV)
    for use_ids in (ids, inp["draft_ids"]):   # the drafted ids, then unrelated ones
        n0, y0, f0 = (t.clone() for t in v(inp["target"], inp["draft"], use_ids,
                                           inp["u_accept"], inp["u_final"]))
        n1, y1, f1 = v.drafted(inp["target"], inp["draft"], use_ids, inp["u_accept"],
                               inp["u_final"], wss)
        torch.cuda.synchronize()
        assert torch.equal(n0, n1) and torch.equal(y0, y1) and torch.equal(f0, f1)
        rn, ry, rf = O.rejection_sample(_np(inp["target"]), _np(inp["draft"]),
                                        use_ids.cpu().numpy(), _np(inp["u_accept"]),
                                        _np(inp["u_final"]), T, tp, tk)
        assert np.array_equal(n1.cpu().numpy(), rn) and np.array_equal(y1.cpu().numpy(), ry)
        assert np.array_equal(f1.cpu().numpy(), rf)


def test_drafted_rejects_mismatched_draft_statistics():
    B, k, V, T, tp = 8, 2, 4096, 0.8, 0.95
    inp = verify_inputs(B, k, V, seed=5, device=DEV, temperature=T, top_p=tp)
    ids, wss = _draft_steps(inp["draft"], 0.9, tp, 0, 3, k, B, V)   # another temperature
    v = Verifier(B, k, V, torch.bfloat16, temperature=T, top_p=tp, device=DEV)
    _, y, f = v.drafted(inp["target"], inp["draft"], ids, inp["u_accept"], inp["u_final"], wss)
    assert bool(((f & FLAG_WORKSPACE) != 0).all())
    # and the workspace stays usable: the next plain call is exact
    n, y, f = v(inp["target"], inp["draft"], ids, inp["u_accept"], inp["u_final"])
    rn, ry, rf = O.rejection_sample(_np(inp["target"]), _np(inp["draft"]), ids.cpu().numpy(),
                                    _np(inp["u_accept"]), _np(inp["u_final"]), T, tp, 0)
    assert np.array_equal(n.cpu().numpy(), rn) and np.array_equal(y.cpu().numpy(), ry)


def test_drafted_graph_replays():
    B, k, V, T, tp = 32, 4, 151936, 0.8, 0.95
    inp = verify_inputs(B, k, V, seed=9, device=DEV, temperature=T, top_p=tp)
    ids, wss = _draft_steps(inp["draft"], T, tp, 0, 4, k, B, V)
    v = Verifier(B, k, V, torch.bfloat16, temperature=T, top_p=tp, device=DEV)
    want = [t.clone() for t in v(inp["target"], inp["draft"], ids, inp["u_accept"], inp["u_final"])]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        v.drafted(inp["target"], inp["draft"], ids, inp["u_accept"], inp["u_final"], wss)
    for _ in range(3):
        v.n_acc.fill_(-3)
        g.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip((v.n_acc, v.y, v.flags), want))
        v(inp["target"], inp["draft"], ids, inp["u_accept"], inp["u_final"])   # eager between

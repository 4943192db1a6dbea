"""The fused verify's bounded wait, made to give up from the host.

SDX_VERIFY_WAIT_TICKS=0 (read at each launch) lets every draw workgroup poll its
batch row's arrivals once: a row whose statistics are not all in at that moment
gives up. Every kernel still exits normally (row workgroups never wait). Then:
* every row either equals the oracle or is flagged SDX_FLAG_WORKSPACE with y -1;
* the next call on the same workspace flags every row (the header is marked);
* after the workspace is prepared again, the call equals the oracle.
"""
import os

import numpy as np
import pytest
import torch

from oracle import sampling as O
from specdec.sampling import FLAG_WORKSPACE, Verifier
from specdec.workloads import verify_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().float().cpu().numpy()


def _run(v, inp):
    n, y, f = v(inp["target"], inp["draft"], inp["draft_ids"], inp["u_accept"], inp["u_final"])
    torch.cuda.synchronize()
    return n.cpu().numpy().copy(), y.cpu().numpy().copy(), f.cpu().numpy().copy()


def test_wait_give_up_flags_then_marks_workspace():
    B, k, V, T, tp = 64, 4, 151936, 0.8, 0.95
    print(f"[giveup] B={B} k={k} V={V}", flush=True)
    inp = verify_inputs(B, k, V, seed=77, device=DEV, temperature=T, top_p=tp)
    rn, ry, rf = O.rejection_sample(_np(inp["target"]), _np(inp["draft"]),
                                    inp["draft_ids"].cpu().numpy(), _np(inp["u_accept"]),
                                    _np(inp["u_final"]), T, tp, 0)
    v = Verifier(B, k, V, torch.bfloat16, temperature=T, top_p=tp, device=DEV)
    os.environ["SDX_VERIFY_WAIT_TICKS"] = "0"
    try:
        n1, y1, f1 = _run(v, inp)
    finally:
        del os.environ["SDX_VERIFY_WAIT_TICKS"]
    flagged = (f1 & FLAG_WORKSPACE) != 0
    print(f"[giveup] rows given up: {int(flagged.sum())} of {B}", flush=True)
    assert flagged.any(), "no draw gave up at a zero wait bound"
    assert np.all(y1[flagged] == -1)
    ok = ~flagged
    assert np.array_equal(n1[ok], rn[ok]) and np.array_equal(y1[ok], ry[ok])
    assert np.array_equal(f1[ok], rf[ok])
    # the header is marked: a normal call now flags every row
    n2, y2, f2 = _run(v, inp)
    assert np.all((f2 & FLAG_WORKSPACE) != 0) and np.all(y2 == -1)
    # prepared again, the workspace gives the oracle's result
    v.reset_workspace()
    n3, y3, f3 = _run(v, inp)
    assert np.array_equal(n3, rn) and np.array_equal(y3, ry) and np.array_equal(f3, rf)


CHUNK = 16384  # ids per to_probs output chunk (the output kernel's workgroup)


def _probs_chunks_exact_or_nan(got, ref):
    """Every output chunk equals the oracle bit for bit or is NaN throughout."""
    given_up = 0
    for r in range(got.shape[0]):
        for c0 in range(0, got.shape[1], CHUNK):
            g, e = got[r, c0:c0 + CHUNK], ref[r, c0:c0 + CHUNK]
            nan = np.isnan(g)
            if nan.all():
                given_up += 1
                continue
            assert not nan.any(), f"row {r} chunk {c0 // CHUNK} partly NaN"
            assert np.array_equal(g.view(np.uint32), e.view(np.uint32)), \
                f"row {r} chunk {c0 // CHUNK} differs"
    return given_up


@pytest.mark.parametrize("case", ["zipf", "one_group"])
def test_to_probs_look_back_give_up(case):
    """SDX_PROBS_WAIT_TICKS=0: an output chunk whose row has a partly kept tie group
    polls the earlier chunks' member counts once and gives up (NaN) if one is not
    yet published. Each chunk is then exact or NaN; the next call is exact."""
    from specdec import sampling as S
    from specdec.workloads import zipf_logits
    V, T, tp = 151936, 0.8, 0.95
    if case == "zipf":
        g = torch.Generator(device=DEV).manual_seed(5)
        x = zipf_logits(64, V, g, DEV)
    else:  # one tie group over the whole row, cut by top-p: every chunk holds members
        x = torch.zeros((16, V), dtype=torch.bfloat16, device=DEV)
        tp = 0.5
    print(f"[giveup] to_probs {case} rows={x.shape[0]} V={V}", flush=True)
    ref = O.to_probs(_np(x), T, tp, 0)
    os.environ["SDX_PROBS_WAIT_TICKS"] = "0"
    try:
        got = _np(S.to_probs(x, T, tp, 0))
        torch.cuda.synchronize()
    finally:
        del os.environ["SDX_PROBS_WAIT_TICKS"]
    n = _probs_chunks_exact_or_nan(got, ref)
    print(f"[giveup] chunks given up: {n}", flush=True)
    assert n > 0, "no chunk gave up at a zero wait bound"
    got2 = _np(S.to_probs(x, T, tp, 0))
    assert _probs_chunks_exact_or_nan(got2, ref) == 0


def test_draft_step_wait_give_up_marks_workspace():
    """The one-launch bf16 draft step with SDX_VERIFY_WAIT_TICKS=0: a row whose
    draw blocks did not all find its statistics in gives up (x -1, qx 0,
    conf 0, stop 1); every other row equals the oracle. The workspace is then
    marked: the next step gives up on every row, and a verify that would take
    its statistics over flags its rows. Prepared again, the step is exact."""
    from specdec import _lib
    from specdec.sampling import draft_step
    from specdec.workloads import uniforms, zipf_logits
    B, V, T, tp = 64, 151936, 0.8, 0.95
    g = torch.Generator(device=DEV).manual_seed(91)
    x = zipf_logits(B, V, g, DEV)
    u = uniforms((B,), g, DEV)
    conf0 = 0.3 + 0.7 * uniforms((B,), g, DEV)
    print(f"[giveup] draft step B={B} V={V}", flush=True)
    rx, rq, rconf, rstop = O.draft_step(_np(x), _np(u), T, tp, 0, conf=_np(conf0), tau=0.5,
                                        step=2, min_k=1)
    ws = _lib.workspace(_lib.lib().sdx_draft_step_workspace(B, V, _lib.dtype_code(x)), DEV)

    def step():
        conf = conf0.clone()
        xs, qx, stop = draft_step(x, u, T, tp, 0, conf=conf, tau=0.5, step=2, min_k=1,
                                  workspace=ws)
        torch.cuda.synchronize()
        return (xs.cpu().numpy(), qx.cpu().numpy(), conf.cpu().numpy(), int(stop.item()))

    os.environ["SDX_VERIFY_WAIT_TICKS"] = "0"
    try:
        x1, q1, c1, s1 = step()
    finally:
        del os.environ["SDX_VERIFY_WAIT_TICKS"]
    gave = x1 == -1
    print(f"[giveup] draft rows given up: {int(gave.sum())} of {B}", flush=True)
    assert gave.any(), "no draft row gave up at a zero wait bound"
    assert np.all(q1[gave] == 0.0) and np.all(c1[gave] == 0.0) and s1 == 1
    ok = ~gave
    assert np.array_equal(x1[ok], rx[ok])
    assert np.array_equal(q1[ok].view(np.uint32), rq[ok].view(np.uint32))
    assert np.array_equal(c1[ok].view(np.uint32), rconf[ok].view(np.uint32))
    # marked: every row of the next step gives up ...
    x2, q2, c2, s2 = step()
    assert np.all(x2 == -1) and np.all(q2 == 0.0) and s2 == 1
    # ... and a verify does not take the marked workspace's statistics over
    k = 1
    inp = verify_inputs(B, k, V, seed=92, device=DEV, temperature=T, top_p=tp)
    v = Verifier(B, k, V, torch.bfloat16, temperature=T, top_p=tp, device=DEV)
    draft = x.view(B, 1, V)
    ids = torch.as_tensor(rx, device=DEV).view(B, 1)
    _, _, f3 = v.drafted(inp["target"], draft, ids, inp["u_accept"], inp["u_final"], [ws])
    torch.cuda.synchronize()
    assert np.all((f3.cpu().numpy() & FLAG_WORKSPACE) != 0)
    # prepared again, the step equals the oracle
    _lib.prepare(ws)
    x4, q4, c4, s4 = step()
    assert np.array_equal(x4, rx) and s4 == rstop
    assert np.array_equal(q4.view(np.uint32), rq.view(np.uint32))
    assert np.array_equal(c4.view(np.uint32), rconf.view(np.uint32))

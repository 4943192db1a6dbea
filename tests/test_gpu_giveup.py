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

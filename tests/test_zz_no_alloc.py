"""sdx_verify_noalloc (the verify on the library's own device scratch) against
sdx_verify on a caller workspace: bit-exact n_acc, y and flags on two calls in
a row, the second smaller; replays of a captured call; the scratch prepared
again by itself after a draw's wait gave up; then a request too large for the
scratch."""
import ctypes
import os

import numpy as np
import pytest
import torch

from specdec import _lib
from specdec.workloads import verify_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _outs(B):
    return (torch.empty(B, dtype=torch.int64, device=DEV),
            torch.empty(B, dtype=torch.int64, device=DEV),
            torch.empty(B, dtype=torch.uint8, device=DEV))


def _launch(noalloc, inp, B, k, V, T, tp, outs, ws=None):
    L = _lib.lib()
    n, y, f = outs
    common = (_lib.ptr(inp["target"]), _lib.ptr(inp["draft"]), _lib.BF16, B, k, V,
              _lib.ptr(inp["draft_ids"]), _lib.ptr(inp["u_accept"]), _lib.ptr(inp["u_final"]),
              None, ctypes.c_float(T), ctypes.c_float(tp), 0, _lib.ptr(n), _lib.ptr(y),
              _lib.ptr(f))
    st = _lib.stream_of(inp["target"])
    if noalloc:
        rc = L.sdx_verify_noalloc(*common, st)
    else:
        rc = L.sdx_verify(*common, _lib.ptr(ws), ws.numel(), st)
    _lib.check(rc, "sdx_verify_noalloc" if noalloc else "sdx_verify")


def _call(noalloc, inp, B, k, V, T, tp):
    outs = _outs(B)
    ws = None if noalloc else _lib.workspace(
        _lib.lib().sdx_verify_workspace(B, k, V, _lib.BF16), DEV)
    _launch(noalloc, inp, B, k, V, T, tp, outs, ws)
    torch.cuda.synchronize()
    return tuple(t.cpu().numpy() for t in outs)


def test_noalloc_matches_workspace_verify():
    T, tp, V = 0.8, 0.95, 151936
    for B, k, seed in ((64, 4, 1000), (16, 2, 1001)):   # second call smaller
        print(f"[no_alloc] B={B} k={k} V={V} seed={seed}", flush=True)
        inp = verify_inputs(B, k, V, seed=seed, device=DEV, temperature=T, top_p=tp)
        got = _call(True, inp, B, k, V, T, tp)
        want = _call(False, inp, B, k, V, T, tp)
        for g, w, name in zip(got, want, ("n_acc", "y", "flags")):
            assert np.array_equal(g, w), f"B={B} k={k}: {name} differs"
        assert 0 < got[0].sum() < B * k


def test_noalloc_graph_replays():
    """A call captured in a HIP graph (after an eager call prepared the scratch),
    replayed three times with eager calls of another shape between replays."""
    T, tp, V = 0.8, 0.95, 151936
    B, k = 32, 4
    print(f"[no_alloc] graph B={B} k={k}", flush=True)
    inp = verify_inputs(B, k, V, seed=1002, device=DEV, temperature=T, top_p=tp)
    other = verify_inputs(8, 3, V, seed=1003, device=DEV, temperature=T, top_p=tp)
    want = _call(False, inp, B, k, V, T, tp)
    assert all(np.array_equal(g, w) for g, w in zip(_call(True, inp, B, k, V, T, tp), want))
    outs = _outs(B)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            _launch(True, inp, B, k, V, T, tp, outs)
    torch.cuda.current_stream().wait_stream(s)
    for r in range(3):
        for t in outs:
            t.fill_(-7 if t.dtype == torch.int64 else 255)
        g.replay()
        torch.cuda.synchronize()
        got = tuple(t.cpu().numpy() for t in outs)
        for gg, w, name in zip(got, want, ("n_acc", "y", "flags")):
            assert np.array_equal(gg, w), f"replay {r}: {name} differs"
        _call(True, other, 8, 3, V, T, tp)          # eager work between replays


def test_noalloc_scratch_rearms_after_give_up():
    """SDX_VERIFY_WAIT_TICKS=0 makes draws give up (rows flagged WORKSPACE, the
    scratch header marked); the next call prepares the scratch again by itself."""
    T, tp, V = 0.8, 0.95, 151936
    B, k = 64, 4
    inp = verify_inputs(B, k, V, seed=1004, device=DEV, temperature=T, top_p=tp)
    want = _call(False, inp, B, k, V, T, tp)
    os.environ["SDX_VERIFY_WAIT_TICKS"] = "0"
    try:
        n1, y1, f1 = _call(True, inp, B, k, V, T, tp)
    finally:
        del os.environ["SDX_VERIFY_WAIT_TICKS"]
    flagged = (f1 & 16) != 0
    print(f"[no_alloc] rows given up: {int(flagged.sum())}", flush=True)
    assert flagged.any() and np.all(y1[flagged] == -1)
    got = _call(True, inp, B, k, V, T, tp)
    for g, w, name in zip(got, want, ("n_acc", "y", "flags")):
        assert np.array_equal(g, w), f"after the give-up: {name} differs"


def test_noalloc_rejects_requests_beyond_its_scratch():
    L = _lib.lib()
    B, k, V = 256, 8, 151936
    n = torch.empty(B, dtype=torch.int64, device=DEV)
    x = torch.empty(8, dtype=torch.bfloat16, device=DEV)
    rc = L.sdx_verify_noalloc(_lib.ptr(x), _lib.ptr(x), _lib.BF16, B, k, V, _lib.ptr(n),
                              _lib.ptr(x), _lib.ptr(x), None, ctypes.c_float(0.8),
                              ctypes.c_float(0.95), 0, _lib.ptr(n), _lib.ptr(n), _lib.ptr(n),
                              _lib.stream_of(x))
    assert rc == -4
    assert b"scratch" in L.sdx_last_error()

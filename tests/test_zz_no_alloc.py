"""sdx_verify_noalloc (the verify on the library's own device scratch) against
sdx_verify on a caller workspace: bit-exact n_acc, y and flags on two calls in
a row, the second smaller, then a request too large for the scratch."""
import ctypes

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


def _call(noalloc, inp, B, k, V, T, tp):
    L = _lib.lib()
    n, y, f = _outs(B)
    common = (_lib.ptr(inp["target"]), _lib.ptr(inp["draft"]), _lib.BF16, B, k, V,
              _lib.ptr(inp["draft_ids"]), _lib.ptr(inp["u_accept"]), _lib.ptr(inp["u_final"]),
              None, ctypes.c_float(T), ctypes.c_float(tp), 0, _lib.ptr(n), _lib.ptr(y),
              _lib.ptr(f))
    st = _lib.stream_of(inp["target"])
    if noalloc:
        rc = L.sdx_verify_noalloc(*common, st)
    else:
        ws = _lib.workspace(L.sdx_verify_workspace(B, k, V, _lib.BF16), DEV)
        rc = L.sdx_verify(*common, _lib.ptr(ws), ws.numel(), st)
    _lib.check(rc, "sdx_verify_noalloc" if noalloc else "sdx_verify")
    torch.cuda.synchronize()
    return tuple(t.cpu().numpy() for t in (n, y, f))


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

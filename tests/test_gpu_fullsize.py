"""GPU parity at the workloads' full sizes.

* Greedy verify B=256, k=8, V=151936 bf16 (the greedy-verify workload) with
  tied maxima planted across rows, through all three entry points that take
  T = 0: sdx_verify_greedy, sdx_verify and sdx_verify_ragged.
* Rows split over several blocks (the rows past the last whole multiple of
  the CU count): one workspace reused by calls of different row counts, and
  the same under graph replay.
* A workspace that sdx_workspace_init never prepared: rows that would use the
  split counters are flagged, every other row still equals the oracle.

The oracle (numpy) is slow on 151936-wide rows (~50 ms per row at T > 0), so
the sampled cases check every batch row whose rows are split plus a few
others against it; the GPU runs the whole batch.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import sampling as O
from specdec import _lib
from specdec import sampling as S
from specdec.workloads import greedy_inputs, ragged_verify_inputs, verify_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"
V = 151936


def _np(t):
    return t.detach().float().cpu().numpy()


def _cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


# ---------------------------------------------------------------- greedy, full size
def _greedy_with_ties(seed):
    B, k = 256, 8
    inp = greedy_inputs(B, k, V, seed=seed, device=DEV)
    tgt = inp["target"].clone()
    ids = inp["draft_ids"].clone()
    rng = np.random.default_rng(seed)
    # every 7th target row gets its maximum at two places far apart; a drafted
    # token at the later copy must be rejected, at the earlier one accepted
    flat = tgt.view(-1, V)
    for r in range(0, B * (k + 1), 7):
        j1, j2 = sorted(rng.choice(V, 2, replace=False).tolist())
        top = flat[r].float().max() + 1.0
        flat[r, j1] = top
        flat[r, j2] = top
        b, i = divmod(r, k + 1)
        if i < k:
            ids[b, i] = j2 if (r // 7) % 2 else j1
    # a row whose ties sit in one 16-byte group and one at the row's last id
    flat[3, 8:16] = flat[3].float().max() + 2.0
    flat[5, V - 1] = flat[5].float().max() + 2.0
    flat[5, 0] = flat[5, V - 1]
    return tgt, ids, inp["u_accept"]


def test_greedy_verify_b256_k8_full_vocab():
    B, k = 256, 8
    tgt, ids, ua = _greedy_with_ties(2000)
    uf = torch.zeros(B, dtype=torch.float32, device=DEV)
    rn, ry, rf = O.greedy_verify(_np(tgt), ids.cpu().numpy(), _np(ua))
    assert rn.min() >= 0 and 0 < (rn == k).sum() < B     # every outcome class present

    def check(res, what):
        for got, want, name in zip(res, (rn, ry, rf), ("n_acc", "y", "flags")):
            g = got.cpu().numpy()
            assert np.array_equal(g, want), f"{what}: {name} differs at {np.flatnonzero(g != want)[:8]}"

    check(S.rejection_sample(tgt, None, ids, ua, uf, temperature=0.0), "sdx_verify_greedy")
    # sdx_verify at T = 0 (its greedy branch), called through the C ABI
    L = _lib.lib()
    n = torch.empty(B, dtype=torch.int64, device=DEV)
    y = torch.empty(B, dtype=torch.int64, device=DEV)
    f = torch.empty(B, dtype=torch.uint8, device=DEV)
    ws = _lib.workspace(L.sdx_verify_workspace(B, k, V, _lib.BF16), DEV)
    rc = L.sdx_verify(_lib.ptr(tgt), _lib.ptr(tgt), _lib.BF16, B, k, V, _lib.ptr(ids),
                      _lib.ptr(ua), _lib.ptr(uf), None, ctypes.c_float(0.0), ctypes.c_float(1.0), 0,
                      _lib.ptr(n), _lib.ptr(y), _lib.ptr(f), _lib.ptr(ws), ws.numel(),
                      _lib.stream_of(tgt))
    _lib.check(rc, "sdx_verify T=0")
    check((n, y, f), "sdx_verify")
    # per-row k at T = 0, every row at k = 8
    cu = torch.arange(B + 1, device=DEV, dtype=torch.int64) * k
    check(S.rejection_sample_ragged(tgt.view(-1, V), None, ids.reshape(-1), ua.reshape(-1), uf, cu,
                                    k_max=k, temperature=0.0), "sdx_verify_ragged")


def test_greedy_ragged_full_vocab_mixed_k():
    """T = 0 with per-row k from 0 to 8 at V = 151936, ties planted in targets."""
    ks = [(5 * b) % 9 for b in range(40)]
    inp = ragged_verify_inputs(len(ks), V, seed=77, device=DEV, temperature=0.0, top_p=1.0,
                               top_k=0, k=ks)
    tgt = inp["target"].clone()
    rng = np.random.default_rng(3)
    for r in range(0, tgt.shape[0], 5):
        j1, j2 = sorted(rng.choice(V, 2, replace=False).tolist())
        tgt[r, j1] = tgt[r, j2] = tgt[r].float().max() + 0.5
    n, y, f = S.rejection_sample_ragged(tgt, None, inp["draft_ids"], inp["u_accept"],
                                        inp["u_final"], inp["cu_k"], k_max=8, temperature=0.0)
    rn, ry, rf = O.rejection_sample_ragged(_np(tgt), None, inp["draft_ids"].cpu().numpy(),
                                           _np(inp["u_accept"]), _np(inp["u_final"]),
                                           inp["cu_k"].cpu().numpy(), 0.0)
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)


# ---------------------------------------------------------------- split rows
def _split_batch_rows(cu, cus):
    """Batch rows with a target or draft row past the last whole multiple of the
    CU count (rows split over blocks when 2 <= cus // rest), in a ragged call
    whose rows are numbered targets first, then drafts."""
    ks = np.diff(cu)
    B = ks.size
    ntgt = int(ks.sum()) + B
    rows = ntgt + int(ks.sum())
    nwhole = rows // cus * cus
    rest = rows - nwhole
    if rest == 0 or cus // rest < 2:
        return [], rows
    out = []
    for b in range(B):
        t_last = int(cu[b]) + b + int(ks[b])
        d_last = ntgt + int(cu[b]) + int(ks[b]) - 1
        if t_last >= nwhole or (ks[b] > 0 and d_last >= nwhole):
            out.append(b)
    return out, rows


def _oracle_subset(inp, sel, T, tp, tk):
    """The ragged oracle on batch rows `sel` only, repacked."""
    cu = inp["cu_k"].cpu().numpy()
    ks = np.diff(cu)
    t_rows, d_rows = [], []
    for b in sel:
        t_rows += list(range(int(cu[b]) + b, int(cu[b]) + b + int(ks[b]) + 1))
        d_rows += list(range(int(cu[b]), int(cu[b]) + int(ks[b])))
    sub_cu = np.concatenate([[0], np.cumsum(ks[sel])]).astype(np.int64)
    d_idx = torch.tensor(d_rows, dtype=torch.int64, device=DEV)
    return O.rejection_sample_ragged(
        _np(inp["target"][torch.tensor(t_rows, device=DEV)]), _np(inp["draft"][d_idx]),
        inp["draft_ids"][d_idx].cpu().numpy(), _np(inp["u_accept"][d_idx]),
        _np(inp["u_final"][torch.tensor(sel, device=DEV)]), sub_cu, T, tp, tk)


def _ks_for_rows(B, rows, seed):
    """k_b in [1, 8] with sum(2 k_b + 1) == rows."""
    total = (rows - B) // 2
    assert (rows - B) % 2 == 0 and B <= total <= 8 * B
    rng = np.random.default_rng(seed)
    ks = np.ones(B, np.int64)
    while ks.sum() < total:
        b = int(rng.integers(B))
        if ks[b] < 8:
            ks[b] += 1
    return ks.tolist()


def _check_subset(res, inp, sel, T, tp, tk):
    rn, ry, rf = _oracle_subset(inp, sel, T, tp, tk)
    idx = np.asarray(sel)
    for got, want, name in zip(res, (rn, ry, rf), ("n_acc", "y", "flags")):
        g = got.cpu().numpy()[idx]
        assert np.array_equal(g, want), f"{name} differs for batch rows {idx[g != want][:8]}"


def test_split_rows_workspace_reused_across_row_counts():
    """One workspace, two ragged calls at B=128 whose row counts (1060, then
    1100 rows: 36 and 76 rows split over blocks on 256 CUs) put the split rows
    at different places; each checked against the oracle on every batch row
    touching a split row plus four others. A third call repeats the first."""
    cus = _cus()
    B, T, tp, tk = 128, 0.7, 0.9, 50
    inps = [ragged_verify_inputs(B, V, seed=900 + i, device=DEV, k=_ks_for_rows(B, rows, i))
            for i, rows in enumerate((1060, 1100))]
    need = max(_lib.lib().sdx_verify_ragged_workspace(B, x["target"].shape[0], V, _lib.BF16)
               for x in inps)
    ws = _lib.workspace(need, DEV)
    for i in (0, 1, 0):
        inp = inps[i]
        split, _ = _split_batch_rows(inp["cu_k"].cpu().numpy(), cus)
        if cus == 256:
            assert split, "the call should split rows on a 256-CU device"
        sel = sorted(set(split) | {0, 1, B // 2, B - 1 - len(split)})
        res = S.rejection_sample_ragged(inp["target"], inp["draft"], inp["draft_ids"],
                                        inp["u_accept"], inp["u_final"], inp["cu_k"], k_max=8,
                                        temperature=T, top_p=tp, top_k=tk, workspace=ws)
        _check_subset(res, inp, sel, T, tp, tk)


def test_split_rows_graph_replays():
    """Per-row k with split rows (B=48, 560 rows: 48 split on 256 CUs) captured in
    a graph on a prepared workspace; replays over two input sets of one row
    layout, with eager calls between, checked against the oracle."""
    cus = _cus()
    B, T, tp, tk = 48, 0.7, 0.9, 50
    ks = _ks_for_rows(B, 560, 5)
    names = ("target", "draft", "draft_ids", "u_accept", "u_final", "cu_k")
    sets = [ragged_verify_inputs(B, V, seed=s, device=DEV, k=ks) for s in (31, 32)]
    split, _ = _split_batch_rows(sets[0]["cu_k"].cpu().numpy(), cus)
    sel = sorted(set(split) | {0, B // 3})
    ref = [_oracle_subset(x, sel, T, tp, tk) for x in sets]
    static = {n: sets[0][n].clone() for n in names}
    ws = _lib.workspace(_lib.lib().sdx_verify_ragged_workspace(B, sum(ks) + B, V, _lib.BF16), DEV)
    out = (torch.empty(B, dtype=torch.int64, device=DEV),
           torch.empty(B, dtype=torch.int64, device=DEV),
           torch.empty(B, dtype=torch.uint8, device=DEV))
    idx = np.asarray(sel)

    def call(src):
        return S.rejection_sample_ragged(src["target"], src["draft"], src["draft_ids"],
                                         src["u_accept"], src["u_final"], src["cu_k"],
                                         k_max=max(ks), temperature=T, top_p=tp, top_k=tk,
                                         workspace=ws, out=out)

    def check(res, i):
        for got, want in zip(res, ref[i]):
            assert np.array_equal(got.cpu().numpy()[idx], want)

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


def test_unprepared_workspace_flags_split_rows():
    """A zero-filled workspace that sdx_workspace_init never prepared: no batch
    row whose result depends on the workspace's counters comes back silently
    wrong. The rows split over blocks do not trust them, so their batch rows
    carry FLAG_WORKSPACE; the one-launch verify (whose draws wait on counters)
    flags every batch row; every batch row not flagged equals the oracle."""
    cus = _cus()
    B, k, T, tp = 64, 4, 0.8, 0.95
    inp = verify_inputs(B, k, V, seed=1000, device=DEV, temperature=T, top_p=tp)
    L = _lib.lib()
    ws = torch.zeros(L.sdx_verify_workspace(B, k, V, _lib.BF16), dtype=torch.uint8, device=DEV)
    n = torch.empty(B, dtype=torch.int64, device=DEV)
    y = torch.empty(B, dtype=torch.int64, device=DEV)
    f = torch.empty(B, dtype=torch.uint8, device=DEV)
    rc = L.sdx_verify(_lib.ptr(inp["target"]), _lib.ptr(inp["draft"]), _lib.BF16, B, k, V,
                      _lib.ptr(inp["draft_ids"]), _lib.ptr(inp["u_accept"]),
                      _lib.ptr(inp["u_final"]), None, ctypes.c_float(T), ctypes.c_float(tp), 0,
                      _lib.ptr(n), _lib.ptr(y), _lib.ptr(f), _lib.ptr(ws), ws.numel(),
                      _lib.stream_of(ws))
    _lib.check(rc, "sdx_verify")
    cu = np.arange(B + 1, dtype=np.int64) * k
    split, _ = _split_batch_rows(cu, cus)
    fl = f.cpu().numpy()
    flagged = set(np.flatnonzero(fl & 16).tolist())
    assert set(split) <= flagged
    if cus == 256:
        assert len(split) > 0
    ok = [b for b in range(B) if b not in flagged][:6]
    if ok:
        rn, ry, rf = O.rejection_sample(_np(inp["target"][ok]), _np(inp["draft"][ok]),
                                        inp["draft_ids"][ok].cpu().numpy(),
                                        _np(inp["u_accept"][ok]), _np(inp["u_final"][ok]), T, tp,
                                        0)
        assert np.array_equal(n.cpu().numpy()[ok], rn)
        assert np.array_equal(y.cpu().numpy()[ok], ry)
        assert np.array_equal(fl[ok], rf)

"""Residual draws through the record where a partially kept tie group's kept
members run out (sampling.py:5-19 top-p on both rows, engine.py:295-303 the
residual draw), on the GPU against the oracle, bit for bit.

Each batch row's target row holds G ids (random positions) at one logit and
every other id far below, so top-p 0.95 keeps part of that tie group: kept
members are the group's first ids in id order, and one record of the draw
holds both kept and dropped members. The draft row is flat over [-0.5, 0.5],
so its nucleus keeps negative logits, whose keys lie more than 2048 keys below
its maximum: the q values of about half the group's members come from the exp
path below the q table, not from the table. The drafted token is outside the
target's group (target probability 0), so position 0 is rejected and y is
drawn from the residual max(p - q, 0), whose mass is all in the kept members.

The uniforms of most rows are near 1: t = u * total then falls in the record
where the kept members run out, and a member's term missing from that
record's mass (or counted with a wrong q) moves t by about one member's mass,
which moves y. Rows: bf16 (the fused verify kernel) and fp16 (row statistics
and the draw in separate kernels), three group sizes.
"""
import numpy as np
import pytest
import torch

from oracle import sampling as O
from oracle.numerics import uniform_threshold
from specdec.sampling import Verifier, rejection_sample

pytestmark = pytest.mark.gpu
DEV = "cuda"
V = 151936


def _rows(B, G, seed):
    """Target [B, 2, V], draft [B, 1, V] (float32) and drafted ids [B, 1]."""
    rng = np.random.default_rng(seed)
    tgt = np.full((B, 2, V), -20.0, dtype=np.float32)
    drf = rng.uniform(-0.5, 0.5, size=(B, 1, V)).astype(np.float32)
    ids = np.zeros((B, 1), dtype=np.int64)
    for b in range(B):
        grp = rng.choice(V, G, replace=False)
        tgt[b, 0, grp] = 2.0
        tgt[b, 1] = rng.normal(0.0, 3.0, V)
        outside = np.setdiff1d(rng.choice(V, 64, replace=False), grp)
        ids[b, 0] = int(outside[0])
    return tgt, drf, ids


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("G", [300, 1000, 5000])
def test_residual_draw_through_partial_group_record(dtype, G):
    B, T, tp = 8, 1.0, 0.95
    print(f"[partial groups] dtype={dtype} G={G} B={B}", flush=True)
    tgt, drf, ids = _rows(B, G, seed=900 + G)
    tl = torch.from_numpy(tgt).to(DEV, dtype)
    dl = torch.from_numpy(drf).to(DEV, dtype)
    ua = torch.full((B, 1), 0.5, dtype=torch.float32, device=DEV)
    uf = torch.tensor([0.97, 0.985, 0.99, 0.995, 0.999, 0.9995, 0.5, 0.25],
                      dtype=torch.float32, device=DEV)
    di = torch.from_numpy(ids).to(DEV)
    n, y, f = rejection_sample(tl, dl, di, ua, uf, temperature=T, top_p=tp)
    torch.cuda.synchronize()
    f32 = lambda t: t.detach().float().cpu().numpy()
    rn, ry, rf = O.rejection_sample(f32(tl), f32(dl), ids, f32(ua), f32(uf), T, tp, 0)
    # the case is what it is meant to be: every row rejects at position 0 and
    # draws a member of the target's group
    assert (rn == 0).all()
    for b in range(B):
        assert tgt[b, 0, int(ry[b])] == 2.0
    # and it sees a wrong mass of that record (a mistake planted in the oracle):
    # with the term of a kept member whose q value is below the q table left
    # out of the total, y moves in the rows whose u is near 1
    moved = 0
    tn, dn, ufn = f32(tl), f32(dl), f32(uf)
    for b in range(6):
        tb, db = tn[b, 0], dn[b, 0]
        p, q = O.to_probs(tb, T, tp, 0), O.to_probs(db, T, tp, 0)
        grp = np.nonzero(tb == 2.0)[0]
        rec = int(grp[p[grp] > 0].max()) // 2048  # where the kept members run out
        slow = [i for i in grp if i // 2048 == rec and p[i] > 0 and db[i] < 0]
        w = O._residual_weights(p, q)
        tot = int((w >> np.uint64(31)).sum(dtype=np.uint64)) << 31
        tot += int((w & np.uint64((1 << 31) - 1)).sum(dtype=np.uint64))
        cum = np.cumsum(w, dtype=np.uint64)
        for i in slow[:1]:
            t = uniform_threshold(ufn[b], tot - int(w[i]))
            moved += int(np.searchsorted(cum, np.uint64(t), side="right")) != int(ry[b])
    assert moved >= 3, moved
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry), (y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)
    if dtype == torch.bfloat16:  # the prepared path, same results
        ver = Verifier(B, 1, V, dtype, temperature=T, top_p=tp, device=DEV)
        n2, y2, f2 = ver(tl, dl, di, ua, uf)
        torch.cuda.synchronize()
        assert np.array_equal(n2.cpu().numpy(), rn)
        assert np.array_equal(y2.cpu().numpy(), ry)
        assert np.array_equal(f2.cpu().numpy(), rf)

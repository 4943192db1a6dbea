"""Pins for `oracle/kvcache.py` and `oracle/controller.py`.

KV: the invariants of the reference's `tests/test_kv_rollback.py:50-90`
(lengths after rollback, rollback below zero raises, stale tail unreachable
through the mask) plus paged == contiguous by brute force.
Controller: the brute-force and monotonicity checks of
`tests/test_controller.py:45-83`.
"""
import numpy as np
import pytest

from oracle import controller as C
from oracle import kvcache as K


def test_rollback_lengths_and_error():
    plen = np.array([7, 5, 6])
    keep = np.array([4, 1, 2])
    lengths = K.advance(plen, 4)
    lengths = K.rollback(lengths, 4 - keep)
    assert lengths.tolist() == (plen + keep).tolist()
    with pytest.raises(RuntimeError, match="below zero"):
        K.rollback(lengths, lengths + 1)


def test_stale_tail_is_masked():
    rs = np.random.RandomState(0)
    B, H, Cap, D, q = 3, 2, 32, 4, 3
    lengths = np.array([5, 9, 2])
    mask = K.attn_mask(lengths, q, neg=-1e30)
    assert mask.shape == (B, 1, q, lengths.max() + q)
    for b in range(B):
        for j in range(q):
            allowed = np.nonzero(mask[b, 0, j] == 0)[0]
            assert allowed.tolist() == list(range(lengths[b] + j + 1))
    assert K.attn_mask(np.array([4, 4]), 2, neg=-1.0) is None
    # writing garbage past every row's live length + q never lands in an allowed slot
    keys = rs.randn(B, H, Cap, D)
    for b in range(B):
        keys[b, :, lengths[b] + q:] = 99.0
        allowed = mask[b, 0] == 0
        assert not np.any(keys[b, :, :allowed.shape[1]][:, allowed.any(0)] == 99.0)


def test_ragged_update_positions():
    B, H, Cap, D, q = 2, 2, 16, 3, 4
    keys = np.zeros((B, H, Cap, D))
    vals = np.zeros((B, H, Cap, D))
    lengths = np.array([3, 7])
    kn = np.arange(B * H * q * D, dtype=float).reshape(B, H, q, D) + 1
    K.ragged_update(keys, vals, lengths, kn, -kn)
    for b in range(B):
        assert np.array_equal(keys[b, :, lengths[b]:lengths[b] + q], kn[b])
        assert np.all(keys[b, :, :lengths[b]] == 0)
    assert K.positions(lengths, q).tolist() == [[3, 4, 5, 6], [7, 8, 9, 10]]


def test_paged_equals_contiguous():
    rs = np.random.RandomState(1)
    B, H, D, bs, q = 4, 2, 8, 16, 5
    lengths = rs.randint(0, 60, B)
    nblk = (lengths.max() + q + bs - 1) // bs
    perm = rs.permutation(B * nblk)
    bt = perm.reshape(B, nblk).astype(np.int32)
    kp = rs.randn(B * nblk, bs, H, D).astype(np.float32)
    vp = rs.randn(B * nblk, bs, H, D).astype(np.float32)
    kn = rs.randn(B, q, H, D).astype(np.float32)
    vn = rs.randn(B, q, H, D).astype(np.float32)
    before = [K.paged_gather(kp, bt, b, int(lengths[b]), bs) for b in range(B)]
    K.paged_append(kp, vp, bt, lengths, kn, vn, bs)
    for b in range(B):
        g = K.paged_gather(kp, bt, b, int(lengths[b]) + q, bs)
        assert np.array_equal(g[:lengths[b]], before[b])
        assert np.array_equal(g[lengths[b]:], kn[b])


def test_slot_mapping_overflow():
    bt = np.array([[3, 5, 7], [2, 4, 6]], np.int32)
    pos, slots = K.slot_mapping(bt, np.array([17, 40]), block_size=16, max_model_len=40)
    assert pos.tolist() == [17, 0]
    assert slots.tolist() == [5 * 16 + 1, -1]


def test_best_k_brute_force_and_monotone():
    for a in (0.3, 0.55, 0.7, 0.9):
        for c in (0.05, 0.12, 0.25):
            bf = max(range(1, 9), key=lambda k: C.expected_speedup(k, a, c))
            assert C.best_k(a, c, 8) == bf
    assert all(C.best_k(a, 0.15) <= C.best_k(a + 0.05, 0.15) for a in (0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9))
    assert all(C.best_k(0.85, c) >= C.best_k(0.85, c + 0.05) for c in (0.05, 0.1, 0.15, 0.2))
    assert C.best_k(0.05, 0.3) == 1
    assert C.best_k(0.98, 0.05, 8) == 8
    for a in (0.6, 0.78, 0.9):
        for c in (0.15, 0.5, 1.0, 1.6):
            assert C.best_k(a, c, 8, 1) >= C.best_k(a, c, 8, 0)
    assert abs(C.expected_speedup(3, 1.0, 0.1) - 4 / 1.4) < 1e-12

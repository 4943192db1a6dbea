"""CPU pins of the verify-attention oracle (oracle/attention.py).

The oracle is pinned against torch's scaled_dot_product_attention (CPU, fp64)
on the same keys gathered densely with an explicit boolean mask built from the
reference's rule s <= lengths[b] + j (specdec/kvcache.py:155), and against a
closed form: a single visible key returns its value row exactly.
"""
import numpy as np
import pytest
import torch

from oracle import attention as A


def _case(B, hq, hkv, d, bs, seed):
    rng = np.random.default_rng(seed)
    qb = rng.integers(1, 6, size=B)
    ctx = rng.integers(0, 70, size=B)
    kv_len = ctx + qb
    pages = (kv_len + bs - 1) // bs
    nb = int(pages.sum()) + 3
    perm = rng.permutation(nb)
    bt = np.full((B, int(pages.max())), -1, np.int64)
    o = 0
    for b in range(B):
        bt[b, :pages[b]] = perm[o:o + pages[b]]
        o += pages[b]
    k_pool = rng.standard_normal((nb, bs, hkv * d))
    v_pool = rng.standard_normal((nb, bs, hkv * d))
    cu = np.concatenate([[0], np.cumsum(qb)])
    q = rng.standard_normal((int(cu[-1]), hq, d))
    return q, cu, k_pool, v_pool, bt, kv_len


@pytest.mark.parametrize("hq,hkv", [(4, 1), (8, 2), (6, 6)])
def test_oracle_matches_torch_sdpa(hq, hkv):
    d, bs = 16, 4
    q, cu, kp, vp, bt, kv_len = _case(5, hq, hkv, d, bs, seed=hq * 10 + hkv)
    scale = 1.0 / np.sqrt(d)
    out = A.verify_attention_paged(q, cu, kp, vp, bt, kv_len, hq, hkv, scale)
    group = hq // hkv
    for b in range(len(kv_len)):
        n, q0, q1 = int(kv_len[b]), int(cu[b]), int(cu[b + 1])
        qb = q1 - q0
        K = torch.from_numpy(A.gather_row(kp, bt[b], n, hkv, d)).permute(1, 0, 2)   # [hkv, n, d]
        V = torch.from_numpy(A.gather_row(vp, bt[b], n, hkv, d)).permute(1, 0, 2)
        K = K.repeat_interleave(group, 0)
        V = V.repeat_interleave(group, 0)
        Q = torch.from_numpy(q[q0:q1]).permute(1, 0, 2)                            # [hq, qb, d]
        s = torch.arange(n)[None, :]
        j = torch.arange(qb)[:, None]
        mask = s <= (n - qb) + j                                                   # kvcache.py:155
        ref = torch.nn.functional.scaled_dot_product_attention(Q, K, V, attn_mask=mask,
                                                               scale=scale)
        np.testing.assert_allclose(out[q0:q1], ref.permute(1, 0, 2).numpy(), rtol=1e-10,
                                   atol=1e-10)


def test_oracle_single_visible_key_returns_its_value():
    d, bs, hq, hkv = 8, 4, 2, 1
    rng = np.random.default_rng(3)
    kp = rng.standard_normal((2, bs, hkv * d))
    vp = rng.standard_normal((2, bs, hkv * d))
    bt = np.array([[1, 0]])
    q = rng.standard_normal((1, hq, d))
    out = A.verify_attention_paged(q, np.array([0, 1]), kp, vp, bt, np.array([1]), hq, hkv, 0.3)
    np.testing.assert_allclose(out[0, 0], vp[1, 0, :d])
    np.testing.assert_allclose(out[0, 1], vp[1, 0, :d])

"""Oracle of the verify attention: one layer of the target's multi-query
attention in a verify forward.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`).

The reference runs HF Qwen3 attention with `attn_implementation="sdpa"`
(`bench/bench_engine.py:170-174`) over its RaggedCache: the k+1 new positions
of row b are written at slots lengths[b] + j (`specdec/kvcache.py:61-74`) and
attend through the additive mask of `specdec/kvcache.py:138-162` (slot s is
visible to query j iff s <= lengths[b] + j); query head h reads KV head
h // (Hq / Hkv) (transformers' `repeat_kv`). This restatement takes the paged
layout of `sdx_kv_append_paged` (pool [num_blocks, block_size, Hkv * D], one
block table) and computes softmax(q k^T * scale) v in float64.
"""
import numpy as np


def gather_row(pool, block_table_row, n, hkv, d):
    """Keys (or values) of one row's first n positions: [n, hkv, d] float64."""
    bs = pool.shape[1]
    pos = np.arange(n)
    pages = np.asarray(block_table_row, np.int64)[pos // bs]
    return pool[pages, pos % bs].reshape(n, hkv, d).astype(np.float64)


def verify_attention_paged(q, cu_q, k_pool, v_pool, block_table, kv_len, hq, hkv, scale):
    """q [T, hq, d] (any float), cu_q [B+1], pools [num_blocks, bs, hkv * d],
    block_table [B, max_blocks], kv_len [B] (keys per row, new positions
    included) -> out [T, hq, d] float64."""
    q = np.asarray(q, np.float64)
    T, _, d = q.shape
    group = hq // hkv
    out = np.zeros((T, hq, d), np.float64)
    for b in range(len(cu_q) - 1):
        q0, q1 = int(cu_q[b]), int(cu_q[b + 1])
        qb, n = q1 - q0, int(kv_len[b])
        base = n - qb                                   # lengths[b] before the new positions
        K = gather_row(k_pool, block_table[b], n, hkv, d)
        Vv = gather_row(v_pool, block_table[b], n, hkv, d)
        for j in range(qb):
            vis = base + j + 1                          # kvcache.py:155: s <= lengths[b] + j
            for h in range(hq):
                kh = h // group                         # repeat_kv
                s = (K[:vis, kh, :] @ q[q0 + j, h]) * scale
                p = np.exp(s - s.max())
                out[q0 + j, h] = (p / p.sum()) @ Vv[:vis, kh, :]
    return out

"""Oracle restatement of the bookkeeping at the end of a speculative round,
`specdec/engine.py:305-340`.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`).
"""
import numpy as np


def round_commit(n_acc, y, draft_ids, k, done, out, eos_ids, max_new, cu_k=None):
    """Row b drafted k_b tokens (k, or cu_k[b+1] - cu_k[b]) and accepted n_acc[b]:
    the caches drop max(0, k_b - n_acc[b]) positions (`engine.py:310-312`);
    unless done, its accepted drafts then y[b] are appended to out[b] (a list),
    stopping at an EOS id or at max_new tokens (`engine.py:321-339`).
    Returns (drop [B], done [B] bool, out) with out / done updated."""
    n_acc = np.asarray(n_acc, np.int64)
    B = n_acc.size
    done = np.array(done, bool).copy()
    drop = np.zeros(B, np.int64)
    eos = set(int(e) for e in eos_ids)
    for b in range(B):
        if cu_k is not None:
            kb, base = int(cu_k[b + 1] - cu_k[b]), int(cu_k[b])
            ids = [int(t) for t in np.asarray(draft_ids).reshape(-1)[base:base + kb]]
        else:
            kb = int(k)
            ids = [int(t) for t in np.asarray(draft_ids)[b]]
        drop[b] = max(0, kb - int(n_acc[b]))
        if done[b]:
            continue
        for j in range(int(n_acc[b])):
            out[b].append(ids[j])
            if ids[j] in eos or len(out[b]) >= max_new:
                done[b] = True
                break
        if done[b]:
            continue
        out[b].append(int(y[b]))
        if int(y[b]) in eos or len(out[b]) >= max_new:
            done[b] = True
    return drop, done, out

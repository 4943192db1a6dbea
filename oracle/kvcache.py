"""Oracle restatement of `specdec/kvcache.py` (ragged KV cache) and the paged slot
formula of `vllm_draft_spec/proposer.py:295-314`.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`). Pure index/byte work, so
every comparison against the HIP path is bit-exact.
"""
import numpy as np


def ragged_update(keys, values, lengths, k_new, v_new):
    """`_RaggedLayer.update` (`kvcache.py:61-74`): write q new rows per batch row
    at slots lengths[b] + j of the [B, H, C, D] buffers. In place."""
    B, H, q, D = k_new.shape
    for b in range(B):
        s0 = int(lengths[b])
        keys[b, :, s0:s0 + q, :] = k_new[b]
        values[b, :, s0:s0 + q, :] = v_new[b]


def advance(lengths, q):
    """`RaggedCache.advance` (`kvcache.py:165-168`)."""
    return np.asarray(lengths, np.int64) + int(q)


def rollback(lengths, n):
    """`RaggedCache.rollback` (`kvcache.py:174-190`); raises like the reference."""
    out = np.asarray(lengths, np.int64) - np.asarray(n, np.int64)
    if np.any(out < 0):
        raise RuntimeError("RaggedCache.rollback below zero")
    return out


def positions(lengths, q):
    """`RaggedCache.positions` (`kvcache.py:129-132`)."""
    return np.asarray(lengths, np.int64)[:, None] + np.arange(q, dtype=np.int64)[None, :]


def attn_mask(lengths, q, neg, valid=None):
    """`RaggedCache.attn_mask` (`kvcache.py:138-162`) as a float array
    [B, 1, q, max_len + q]: 0 where slot s <= lengths[b] + j (and s < valid[b]),
    `neg` elsewhere. None when lengths are uniform and there is no pad."""
    lengths = np.asarray(lengths, np.int64)
    if valid is None and lengths.min() == lengths.max():
        return None
    kv = int(lengths.max()) + q
    s = np.arange(kv)[None, None, :]
    j = np.arange(q)[None, :, None]
    allowed = s <= lengths[:, None, None] + j
    if valid is not None:
        allowed &= s < np.asarray(valid, np.int64)[:, None, None]
    return np.where(allowed, 0.0, neg)[:, None, :, :]


def slot_of(block_table, b, pos, block_size):
    """Paged slot of logical position `pos` of row b (`proposer.py:308-312`)."""
    return int(block_table[b, pos // block_size]) * block_size + pos % block_size


def paged_append(k_pool, v_pool, block_table, lengths, k_new, v_new, block_size):
    """Append q positions per row into one layer's paged pools [num_blocks, bs, H, D]
    at logical positions lengths[b] + j. In place."""
    B, q = k_new.shape[0], k_new.shape[1]
    for b in range(B):
        for j in range(q):
            slot = slot_of(block_table, b, int(lengths[b]) + j, block_size)
            k_pool[slot // block_size, slot % block_size] = k_new[b, j]
            v_pool[slot // block_size, slot % block_size] = v_new[b, j]


def paged_gather(pool, block_table, b, length, block_size):
    """Logical positions [0, length) of row b as a contiguous [length, H, D] array."""
    rows = [pool[slot_of(block_table, b, p, block_size) // block_size,
                 slot_of(block_table, b, p, block_size) % block_size] for p in range(length)]
    return np.stack(rows) if rows else pool[:0, 0]


def slot_mapping(block_table, positions, block_size, max_model_len, padding_slot=-1):
    """Drafting-step slot mapping of `proposer.py:295-314`.

    positions [R] are the new positions; rows at or past max_model_len are
    parked at position 0 and get the padding slot (vLLM's PADDING_SLOT_ID,
    imported at `proposer.py:47`; its value is a parameter here). Returns
    (clamped_positions, slots)."""
    pos = np.asarray(positions, np.int64)
    over = pos >= max_model_len
    clamped = np.where(over, 0, pos)
    bt = np.asarray(block_table)
    blk = bt[np.arange(len(pos)), clamped // block_size].astype(np.int64)
    slots = blk * block_size + clamped % block_size
    slots = np.where(over, padding_slot, slots)
    return clamped, slots

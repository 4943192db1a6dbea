"""GPU parity of the KV-cache and proposer kernels against `oracle/kvcache.py`
(bit-exact: pure index and byte work)."""
import numpy as np
import pytest
import torch

from oracle import kvcache as OK
from oracle import sampling as OS
from specdec.kvcache import PagedKVCache, RaggedCache
from specdec.proposer_ops import drafting_slot_mapping, greedy_draft_tokens
from specdec.workloads import kv_inputs, zipf_logits

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_ragged_update_rollback_mask():
    torch.manual_seed(0)
    B, H, Cap, D = 3, 2, 64, 16
    cache = RaggedCache(2, B, Cap, DEV)
    plen = torch.tensor([7, 5, 6])
    k0 = torch.randn(B, H, 7, D, device=DEV, dtype=torch.bfloat16)
    v0 = torch.randn(B, H, 7, D, device=DEV, dtype=torch.bfloat16)
    ks, vs = cache.layers[0].update(k0, v0)
    assert ks.shape == (B, H, 7, D)
    cache.set_lengths(plen)
    keys = np.zeros((B, H, Cap, D), np.float32)
    vals = np.zeros((B, H, Cap, D), np.float32)
    OK.ragged_update(keys, vals, np.zeros(B, np.int64), k0.float().cpu().numpy(),
                     v0.float().cpu().numpy())
    spec_k = torch.randn(B, H, 4, D, device=DEV, dtype=torch.bfloat16)
    spec_v = torch.randn(B, H, 4, D, device=DEV, dtype=torch.bfloat16)
    cache.layers[0].update(spec_k, spec_v)
    OK.ragged_update(keys, vals, plen.numpy(), spec_k.float().cpu().numpy(),
                     spec_v.float().cpu().numpy())
    assert np.array_equal(cache.layers[0].keys.float().cpu().numpy(), keys)
    assert np.array_equal(cache.layers[0].values.float().cpu().numpy(), vals)
    cache.advance(4)
    keep = torch.tensor([4, 1, 2])
    cache.rollback(4 - keep)
    assert cache.lengths.cpu().tolist() == (plen + keep).tolist()
    for dtype in (torch.float32, torch.bfloat16):
        m = cache.attn_mask(3, dtype)
        ref = OK.attn_mask((plen + keep).numpy(), 3, float(torch.finfo(dtype).min))
        assert np.array_equal(m.float().cpu().numpy(), ref.astype(np.float32))
    valid = torch.tensor([3, 9, 8])
    m = cache.attn_mask(2, torch.float32, valid=valid)
    ref = OK.attn_mask((plen + keep).numpy(), 2, float(torch.finfo(torch.float32).min), valid.numpy())
    assert np.array_equal(m.cpu().numpy(), ref.astype(np.float32))
    with pytest.raises(RuntimeError, match="below zero"):
        cache.rollback([100, 0, 0])


def test_ragged_device_rollback_and_overflow_flag():
    B, H, Cap, D = 4, 1, 8, 8
    cache = RaggedCache(1, B, Cap, DEV)
    cache.set_lengths([2, 3, 4, 5])
    cache.rollback_device(torch.tensor([1, 1, 1, 1], device=DEV))
    cache.sync_lengths()
    assert cache.lengths_cpu.tolist() == [1, 2, 3, 4]
    cache.rollback_device(torch.tensor([0, 3, 0, 0], device=DEV))   # row 1 would go negative
    cache.sync_lengths()
    assert cache.lengths_cpu.tolist() == [1, 2, 3, 4]
    assert int(cache.error.item()) == 1
    cache.error.zero_()
    x = torch.ones(B, H, 5, D, device=DEV)                            # 4 + 5 > capacity 8
    cache.layers[0].update(x, x)
    assert int(cache.error.item()) == 1


def test_paged_append_commit_rollback():
    L, B, q, H, D, bs = 4, 8, 5, 8, 128, 16
    inp = kv_inputs(L, B, q, H, D, bs, 20, 100, seed=1, device=DEV)
    c = PagedKVCache(L, B, inp["num_blocks"], bs, H, D, inp["max_blocks"], device=DEV)
    c.block_table.copy_(inp["block_table"])
    c.lengths.copy_(inp["lengths"])
    c.append(inp["staged"])
    c.commit(q)
    c.rollback(q - inp["keep"])
    lengths = inp["lengths"].cpu().numpy()
    assert np.array_equal(c.lengths.cpu().numpy(), lengths + inp["keep"].cpu().numpy())
    bt = inp["block_table"].cpu().numpy()
    staged = inp["staged"].float().cpu().numpy()
    pool = np.zeros((L, 2, inp["num_blocks"], bs, H * D), np.float32)
    for layer in range(L):
        OK.paged_append(pool[layer, 0], pool[layer, 1], bt, lengths, staged[layer, 0],
                        staged[layer, 1], bs)
    assert np.array_equal(c.pool.float().cpu().numpy(), pool)
    assert int(c.error.item()) == 0
    for b in range(B):
        g = c.gather(1, 0, b, int(lengths[b]) + q).float().cpu().numpy()
        assert np.array_equal(g[int(lengths[b]):], staged[1, 0, b])


def test_slot_mapping_and_argmax():
    bt = torch.tensor([[3, 5, 7], [2, 4, 6], [9, 8, 1]], dtype=torch.int32, device=DEV)
    pos = torch.tensor([17, 40, 33], device=DEV)
    cp, slots = drafting_slot_mapping(bt, pos, 16, 40)
    rp, rs = OK.slot_mapping(bt.cpu().numpy(), pos.cpu().numpy(), 16, 40)
    assert np.array_equal(cp.cpu().numpy(), rp)
    assert np.array_equal(slots.cpu().numpy(), rs)
    g = torch.Generator(device=DEV).manual_seed(2)
    x = zipf_logits(37, 151936, g, DEV)
    x[3, :] = 0.0
    x[3, 10] = -0.0
    x[4, [5, 9]] = 50.0                   # exact tie: first index wins
    got = greedy_draft_tokens(x).cpu().numpy()
    assert np.array_equal(got, OS.argmax_first(x.float().cpu().numpy()))
    assert got[3] == 0 and got[4] == 5
    for dt in (torch.float32, torch.float16):
        y = x[:, :4096].to(dt)
        assert np.array_equal(greedy_draft_tokens(y).cpu().numpy(),
                              OS.argmax_first(y.float().cpu().numpy()))

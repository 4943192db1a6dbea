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


def test_ragged_device_rollback_then_advance_without_sync():
    """The engine loop with device counts (`engine.py:248-312`): rollback_device,
    then the next forward's positions / mask / update / advance with no
    sync_lengths in between. Device lengths, mask and written slots equal the
    oracle's; the host mirror is re-read only when asked for."""
    B, H, Cap, D, q = 4, 2, 64, 16, 4
    cache = RaggedCache(1, B, Cap, DEV)
    plen = np.array([7, 5, 6, 9])
    cache.set_lengths(plen)
    keys = np.zeros((B, H, Cap, D), np.float32)
    vals = np.zeros((B, H, Cap, D), np.float32)
    k1 = torch.randn(B, H, q, D, device=DEV, dtype=torch.bfloat16)
    v1 = torch.randn(B, H, q, D, device=DEV, dtype=torch.bfloat16)
    cache.layers[0].update(k1, v1)
    OK.ragged_update(keys, vals, plen, k1.float().cpu().numpy(), v1.float().cpu().numpy())
    cache.advance(q)
    drop = torch.tensor([3, 0, 2, 4], device=DEV)
    cache.rollback_device(drop)                       # no host sync
    assert cache.host_stale
    len1 = OK.rollback(OK.advance(plen, q), drop.cpu().numpy())
    q2 = 3
    assert np.array_equal(cache.positions(q2).cpu().numpy(), OK.positions(len1, q2))
    m = cache.attn_mask(q2, torch.float32)            # built from the device lengths
    neg = float(torch.finfo(torch.float32).min)
    ref = OK.attn_mask(len1, q2, neg)
    kv = ref.shape[-1]
    assert m.shape[-1] >= kv                          # host upper bound of max_len + q2
    assert np.array_equal(m[..., :kv].cpu().numpy(), ref.astype(np.float32))
    assert bool((m[..., kv:] == neg).all())
    k2 = torch.randn(B, H, q2, D, device=DEV, dtype=torch.bfloat16)
    v2 = torch.randn(B, H, q2, D, device=DEV, dtype=torch.bfloat16)
    ks, _ = cache.layers[0].update(k2, v2)            # writes at the rolled-back offsets
    assert ks.shape[2] == m.shape[-1]
    OK.ragged_update(keys, vals, len1, k2.float().cpu().numpy(), v2.float().cpu().numpy())
    cache.advance(q2)                                 # on the device while stale
    assert cache.host_stale
    assert np.array_equal(cache.layers[0].keys.float().cpu().numpy(), keys)
    assert np.array_equal(cache.layers[0].values.float().cpu().numpy(), vals)
    assert np.array_equal(cache.lengths.cpu().numpy(), OK.advance(len1, q2))
    assert cache.lengths_cpu.tolist() == OK.advance(len1, q2).tolist()   # re-read on access
    assert not cache.host_stale and cache.max_len == int(OK.advance(len1, q2).max())
    cache.rollback_device(torch.tensor([1, 1, 1, 1], device=DEV))
    cache.rollback([1, 0, 0, 2])                      # host rollback re-reads first
    assert cache.lengths.cpu().tolist() == (OK.advance(len1, q2) - [2, 1, 1, 3]).tolist()
    assert int(cache.error.item()) == 0


def _checksum(flat, chunk=1 << 28):
    """Sum of an int16 tensor in int64, a chunk at a time (torch would upcast the
    whole tensor at once)."""
    tot = torch.zeros((), dtype=torch.int64, device=flat.device)
    for i in range(0, flat.numel(), chunk):
        tot += flat[i:i + chunk].sum(dtype=torch.int64)
    return int(tot)


def test_paged_append_config4_full_size():
    """The paged-KV workload at full size: 64 layers sharing one block table, B=64,
    lengths ~ U[512, 4096], 5 positions per row, 8 x 128 bf16, block 16 (69 GB of
    pool). The appended slots of every (layer, side, row) equal the staged rows
    byte for byte; a checksum of the whole pool moves by exactly the bytes
    written (no stray writes); lengths after commit + rollback equal len + keep."""
    L, B, q, H, D, bs = 64, 64, 5, 8, 128, 16
    inp = kv_inputs(L, B, q, H, D, bs, 512, 4096, seed=3, device=DEV)
    c = PagedKVCache(L, B, inp["num_blocks"], bs, H, D, inp["max_blocks"], device=DEV)
    c.block_table.copy_(inp["block_table"])
    c.lengths.copy_(inp["lengths"])
    flat = c.pool.view(torch.int16).view(-1)
    flat.random_(-32768, 32767)                       # pre-existing pages: random bytes
    lengths = inp["lengths"].cpu().numpy()
    bt = inp["block_table"].cpu().numpy()
    pos = lengths[:, None] + np.arange(q)[None, :]                        # [B, q]
    slot = bt[np.arange(B)[:, None], pos // bs].astype(np.int64) * bs + pos % bs
    assert pos.min() >= 512 and (pos // bs).max() >= 250    # positions >= 512, block index >= 32
    side_rows = inp["num_blocks"] * bs                                    # rows per (layer, side)
    base = (np.arange(L)[:, None] * 2 + np.arange(2)[None, :]) * side_rows    # [L, 2]
    rows = torch.tensor((base[:, :, None, None] + slot[None, None]).reshape(-1), device=DEV)
    view = c.pool.view(-1, H * D)
    old = view[rows].view(torch.int16)
    before = _checksum(flat) - int(old.sum(dtype=torch.int64))
    c.append(inp["staged"])
    got = view[rows].view(torch.int16)
    staged = inp["staged"].view(torch.int16).reshape(-1, H * D)           # [L, 2, B, q] order
    assert torch.equal(got, staged)
    after = _checksum(flat) - int(staged.sum(dtype=torch.int64))
    assert after == before
    c.commit(q)
    c.rollback(q - inp["keep"])
    assert np.array_equal(c.lengths.cpu().numpy(), lengths + inp["keep"].cpu().numpy())
    assert int(c.error.item()) == 0


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


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("V", [8, 4099, 4096 * 4 + 13, 151936])
def test_argmax_strided_rows_edges(dt, V):
    """sdx_argmax on rows with a padded stride (16-byte aligned, so the packed
    whole-chunk path runs and the last V % 8 elements take the per-element one):
    zeros with a -0, all-equal rows, the maximum in the last element, ties across
    rounds and chunk slots, -inf rows; first index among equal maxima."""
    from specdec import _lib
    ld = (V + 7) // 8 * 8 + 8
    g = torch.Generator(device=DEV).manual_seed(V)
    base = torch.randn((10, ld), generator=g, device=DEV).to(dt)
    x = base[:, :V]
    x[0] = 0.0
    x[0, V // 2] = -0.0
    x[1] = -3.0
    x[2, V - 1] = 100.0
    x[3, [1, V - 2]] = 100.0
    x[4] = -float("inf")
    x[4, V - 1] = -1000.0
    x[5, [V - 1, V // 3, (V // 3) + 4097 if (V // 3) + 4097 < V else 0]] = 50.0
    x[6] = -0.0
    x[7] = -float("inf")
    x[8, [0, V - 1]] = 60.0
    out = torch.empty(10, dtype=torch.int64, device=DEV)
    rc = _lib.lib().sdx_argmax(_lib.ptr(base), _lib.dtype_code(base), 10, V, ld, _lib.ptr(out),
                               _lib.stream_of(base))
    _lib.check(rc, "sdx_argmax")
    want = OS.argmax_first(x.float().cpu().numpy())
    assert np.array_equal(out.cpu().numpy(), want), (out.cpu().numpy(), want)

"""KV caches whose rows roll back independently in O(1), on MI355X.

`RaggedCache` is the drop-in for the reference's `specdec/kvcache.py:87-202`:
one preallocated [B, H_kv, C, D] buffer per layer plus per-row lengths; writes
scatter to each row's own offset (`_RaggedLayer.update`, `kvcache.py:61-74`)
with a HIP kernel, rollback is `lengths -= n`, the additive mask comes from
the lengths (`kvcache.py:138-162`). As in the reference, the host copy of the
lengths is the source of truth when callers pass host lists; `rollback_device`
is the sync-free variant for counts that stay on the device.

`PagedKVCache` is the layout of the vLLM path (`vllm_draft_spec/proposer.py:18-22`):
all layers of the target+draft pair share one block table; a step appends
q candidate positions per row into every layer with one kernel, then commits
and rolls back by per-row counts without touching K/V bytes.
"""
import torch

from . import _lib

try:  # HF integration is optional: the cache works standalone
    from transformers.cache_utils import Cache as _HFCache, CacheLayerMixin as _HFLayer
except Exception:  # pragma: no cover - transformers absent
    _HFCache, _HFLayer = object, object

__all__ = ["RaggedCache", "PagedKVCache"]


class _RaggedLayer(_HFLayer):
    """One layer's preallocated buffer; offsets come from the shared parent."""

    is_sliding = False
    is_compileable = False

    def __init__(self, parent):
        if _HFLayer is not object:
            super().__init__()
        self.parent = parent
        self.keys = None
        self.values = None
        self.is_initialized = False

    def lazy_initialization(self, key_states, value_states=None):
        """`kvcache.py:53-59`: allocate at the first update's dtype/device."""
        p = self.parent
        b, h, _, d = key_states.shape
        self.dtype, self.device = key_states.dtype, key_states.device
        self.keys = torch.zeros(b, h, p.capacity, d, dtype=self.dtype, device=self.device)
        self.values = torch.zeros(b, h, p.capacity, d, dtype=self.dtype, device=self.device)
        self.is_initialized = True

    def update(self, key_states, value_states, *args, **kwargs):
        """Write q new positions per row at lengths[b] + j (`kvcache.py:61-74`).

        Offsets are the lengths before this forward; the parent advances them
        once after every layer has written."""
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        p = self.parent
        _lib.require_gpu(key_states, value_states)
        b, h, q, d = key_states.shape
        kn = key_states.to(self.dtype).contiguous()
        vn = value_states.to(self.dtype).contiguous()
        rc = _lib.lib().sdx_ragged_update(
            _lib.ptr(self.keys), _lib.ptr(self.values), _lib.ptr(kn), _lib.ptr(vn),
            _lib.dtype_code(self.keys), b, h, p.capacity, d, q, _lib.ptr(p.lengths),
            _lib.ptr(p.error), _lib.stream_of(self.keys))
        _lib.check(rc, "RaggedCache.update")
        kv_len = p.kv_len_for(q)
        return self.keys[:, :, :kv_len, :], self.values[:, :, :kv_len, :]

    def get_mask_sizes(self, query_length, *args):
        q = query_length if isinstance(query_length, int) else int(query_length.shape[0])
        return self.parent.kv_len_for(q), 0

    def get_seq_length(self, *args):
        return self.parent.max_len if self.is_initialized else 0

    def get_max_cache_shape(self, *args):
        return self.parent.capacity

    def get_max_length(self, *args):
        return self.parent.capacity


class RaggedCache(_HFCache):
    """Per-row-length KV cache with O(1) rollback (`kvcache.py:87-202`).

    Usage per forward (as the reference):
        pos  = cache.positions(q)
        mask = cache.attn_mask(q, dtype, valid)
        out  = model(input_ids, position_ids=pos, attention_mask=mask,
                     past_key_values=cache, cache_position=cache.cache_position(q))
        cache.advance(q)
    """

    def __init__(self, n_layers, batch_size, capacity, device):
        self.capacity = int(capacity)
        self._batch = int(batch_size)
        self.device = torch.device(device)
        self._lengths_cpu = torch.zeros(self._batch, dtype=torch.long)
        self.lengths = torch.zeros(self._batch, dtype=torch.long, device=self.device)
        # device-side error flag of the scatter / device rollback kernels
        self.error = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.max_len = 0
        self._uniform = True
        # After rollback_device the device lengths are authoritative and the host
        # mirror is stale ("dirty"): max_len is then an upper bound of the true
        # maximum (rollbacks only shrink rows), masks are built on the device from
        # the device lengths, and host-side mutations re-read the lengths first.
        self._dirty = False
        layers = [_RaggedLayer(self) for _ in range(n_layers)]
        if _HFCache is not object:
            super().__init__(layers=layers)
        else:
            self.layers = layers

    @property
    def batch_size(self):
        return self._batch

    @property
    def lengths_cpu(self):
        """Host copy of the row lengths (`kvcache.py:102-113`). After
        `rollback_device` it is re-read from the device first (one sync)."""
        if self._dirty:
            self.sync_lengths()
        return self._lengths_cpu

    @property
    def host_stale(self):
        """True while the device lengths have moved past the host mirror."""
        return self._dirty

    def _push(self):
        """Mirror host lengths to the device (`kvcache.py:118-122`)."""
        self.lengths.copy_(self._lengths_cpu, non_blocking=True)
        self._dirty = False
        self.max_len = int(self._lengths_cpu.max()) if self.batch_size else 0
        self._uniform = bool(int(self._lengths_cpu.min()) == self.max_len) if self.batch_size else True

    # ---- geometry (`kvcache.py:125-162`)
    def kv_len_for(self, q):
        return self.max_len + q

    def positions(self, q):
        ar = torch.arange(q, device=self.device).view(1, q)
        return self.lengths.view(-1, 1) + ar

    def cache_position(self, q):
        return torch.arange(self.max_len, self.max_len + q, device=self.device)

    def attn_mask(self, q, dtype, valid=None):
        """Additive [B, 1, q, kv_len] mask, 0 where s <= lengths[b] + j (and
        s < valid[b]), finfo(dtype).min elsewhere; None when uniform and unpadded.
        While the host mirror is stale the mask is always built (from the device
        lengths) and kv_len is the host's upper bound: the extra columns are masked."""
        if valid is None and self._uniform and not self._dirty:
            return None
        kv_len = self.kv_len_for(q)
        out = torch.empty((self.batch_size, 1, q, kv_len), dtype=dtype, device=self.device)
        v = None if valid is None else valid.to(device=self.device, dtype=torch.long).contiguous()
        rc = _lib.lib().sdx_attn_mask(_lib.ptr(self.lengths), _lib.ptr(v), self.batch_size, q, kv_len,
                                      float(torch.finfo(dtype).min), _lib.dtype_code(out),
                                      _lib.ptr(out), _lib.stream_of(out))
        _lib.check(rc, "RaggedCache.attn_mask")
        return out

    # ---- mutation (`kvcache.py:165-202`)
    def advance(self, q):
        """lengths += q (`kvcache.py:165-168`). While the host mirror is stale the
        device lengths advance in place (no host sync) and max_len stays an upper
        bound."""
        if self._dirty:
            rc = _lib.lib().sdx_kv_advance(_lib.ptr(self.lengths), self.batch_size, int(q),
                                           _lib.stream_of(self.lengths))
            _lib.check(rc, "RaggedCache.advance")
            self.max_len += int(q)
            return
        self._lengths_cpu += int(q)
        self._push()

    def commit(self, q):
        """`advance(q)` under the name the engine and `PagedKVCache` use."""
        self.advance(q)

    def set_lengths(self, lengths):
        self._lengths_cpu.copy_(torch.as_tensor(lengths, dtype=torch.long).cpu())
        self._push()

    def device_rolled_back(self):
        """A kernel (the engine's round commit) moved the device lengths: the host
        mirror is stale until `set_host_lengths` or `sync_lengths`, as after
        `rollback_device`."""
        self._dirty = True
        self._uniform = False

    def set_host_lengths(self, lengths_cpu):
        """Take the device lengths the caller already read back (no sync here)."""
        self._lengths_cpu.copy_(torch.as_tensor(lengths_cpu, dtype=torch.long))
        self._dirty = False
        self.max_len = int(self._lengths_cpu.max()) if self.batch_size else 0
        self._uniform = bool(int(self._lengths_cpu.min()) == self.max_len) if self.batch_size else True

    def rollback(self, n):
        """Drop the last n[b] tokens of row b; raises below zero like the reference."""
        if isinstance(n, int):
            n_cpu = torch.full((self.batch_size,), n, dtype=torch.long)
        elif torch.is_tensor(n):
            n_cpu = n.detach().to("cpu", torch.long)
        else:
            n_cpu = torch.as_tensor(list(n), dtype=torch.long)
        cur = self.lengths_cpu  # re-read first if a device rollback left it stale
        new = cur - n_cpu
        if bool((new < 0).any()):
            raise RuntimeError("RaggedCache.rollback below zero")
        cur.copy_(new)
        self._push()

    def rollback_device(self, n):
        """Sync-free rollback by device counts n [B] (int64). Applies to the device
        lengths; if any row would go negative nothing changes and `self.error` is
        set. The host mirror becomes stale: until `sync_lengths()` (or a host-side
        mutation, which re-reads it) `advance` runs on the device, max_len is an
        upper bound and `attn_mask` is built from the device lengths."""
        _lib.require_gpu(n)
        n = n.to(torch.int64).contiguous()
        rc = _lib.lib().sdx_kv_rollback(_lib.ptr(self.lengths), self.batch_size, _lib.ptr(n),
                                        _lib.ptr(self.error), _lib.stream_of(n))
        _lib.check(rc, "RaggedCache.rollback_device")
        self._dirty = True
        self._uniform = False

    def sync_lengths(self):
        """Re-read device lengths into the host mirror (one device sync)."""
        self._lengths_cpu.copy_(self.lengths.cpu())
        self._dirty = False
        self.max_len = int(self._lengths_cpu.max()) if self.batch_size else 0
        self._uniform = bool(int(self._lengths_cpu.min()) == self.max_len) if self.batch_size else True

    def get_seq_length(self, layer_idx: int = 0):
        return self.max_len

    def reset(self):
        self._lengths_cpu.zero_()
        self._push()
        for layer in self.layers:
            if layer.is_initialized:
                layer.keys.zero_()
                layer.values.zero_()


class PagedKVCache:
    """Paged K/V for L layers sharing one block table (the 36 target + 28 draft
    layers of one vLLM KV group, `proposer.py:18-22`).

    pool: [L, 2, num_blocks, block_size, kv_heads * head_dim] (side 0 = K, 1 = V).
    block_table: [B, max_blocks] int32, filled by the caller's block manager.
    lengths: [B] int64 on the device, the committed length of each row.
    """

    def __init__(self, n_layers, batch_size, num_blocks, block_size, kv_heads, head_dim,
                 max_blocks, dtype=torch.bfloat16, device="cuda"):
        self.n_layers, self.batch_size = int(n_layers), int(batch_size)
        self.num_blocks, self.block_size = int(num_blocks), int(block_size)
        self.row_elems = int(kv_heads) * int(head_dim)
        self.max_blocks = int(max_blocks)
        dev = torch.device(device)
        self.pool = torch.zeros((self.n_layers, 2, self.num_blocks, self.block_size, self.row_elems),
                                dtype=dtype, device=dev)
        self.block_table = torch.full((self.batch_size, self.max_blocks), -1, dtype=torch.int32,
                                      device=dev)
        self.lengths = torch.zeros(self.batch_size, dtype=torch.int64, device=dev)
        self.error = torch.zeros(1, dtype=torch.int32, device=dev)

    def append(self, staged):
        """Write staged [L, 2, B, q, row_elems] at positions lengths[b] + j of every
        layer (does not move the lengths: call `commit(q)` after the step)."""
        _lib.require_gpu(staged)
        L, two, B, q, re = staged.shape
        if (L, two, B, re) != (self.n_layers, 2, self.batch_size, self.row_elems):
            raise ValueError(f"staged must be [{self.n_layers}, 2, {self.batch_size}, q, "
                             f"{self.row_elems}], got {tuple(staged.shape)}")
        st = staged.to(self.pool.dtype).contiguous()
        side = self.num_blocks * self.block_size * self.row_elems
        rc = _lib.lib().sdx_kv_append_paged(
            _lib.ptr(self.pool), 2 * side, side, _lib.ptr(st), _lib.dtype_code(self.pool),
            self.n_layers, self.batch_size, q, self.row_elems, _lib.ptr(self.block_table),
            self.max_blocks, self.block_size, self.num_blocks, _lib.ptr(self.lengths),
            _lib.ptr(self.error), _lib.stream_of(st))
        _lib.check(rc, "PagedKVCache.append")

    def commit(self, q):
        """lengths += q (`kvcache.py:165-168`)."""
        rc = _lib.lib().sdx_kv_advance(_lib.ptr(self.lengths), self.batch_size, int(q),
                                       _lib.stream_of(self.lengths))
        _lib.check(rc, "PagedKVCache.commit")

    def rollback(self, n):
        """lengths -= n (device [B] int64); all-or-nothing, `error` set if any row
        would go negative (`kvcache.py:174-190`)."""
        _lib.require_gpu(n)
        n = n.to(torch.int64).contiguous()
        rc = _lib.lib().sdx_kv_rollback(_lib.ptr(self.lengths), self.batch_size, _lib.ptr(n),
                                        _lib.ptr(self.error), _lib.stream_of(n))
        _lib.check(rc, "PagedKVCache.rollback")

    def slots(self, b, length):
        """Physical slots of logical positions [0, length) of row b (host helper)."""
        pos = torch.arange(length, device=self.block_table.device)
        blk = self.block_table[b, pos // self.block_size].to(torch.int64)
        return blk * self.block_size + pos % self.block_size

    def gather(self, layer, side, b, length):
        """Contiguous [length, row_elems] view of row b's first `length` positions."""
        flat = self.pool[layer, side].reshape(-1, self.row_elems)
        return flat[self.slots(b, length)]

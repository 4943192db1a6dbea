"""Verify attention over the paged KV cache (one layer), on MFMA.

The attention of the target's verify forward: every batch row's k_b + 1 new
positions against the row's cached keys, under the mask of
`specdec/kvcache.py:138-162` (query j of row b sees slot s iff
s <= lengths[b] + j) with grouped-query heads (`repeat_kv`). The reference runs
it as HF SDPA inside the target forward (`bench/bench_engine.py:170-174`,
`specdec/engine.py:273-275`); here it reads the pool that
`PagedKVCache.append` writes, so the new positions' K/V must be appended first.
"""
import math

import torch

from . import _lib

__all__ = ["verify_attention_paged", "attention_workspace"]


def attention_workspace(B, max_q, hq, hkv, block_size, max_blocks, chunk_tokens=0,
                        device="cuda"):
    """A workspace for verify_attention_paged at these sizes (uint8 device tensor)."""
    need = _lib.lib().sdx_verify_attention_workspace(B, int(max_q), hq, hkv, block_size,
                                                     max_blocks, int(chunk_tokens))
    if need == 0:
        _lib.check(-1, "verify_attention workspace query")
    return torch.empty(need, dtype=torch.uint8, device=device)


def verify_attention_paged(q, cu_q, k_pool, v_pool, block_table, kv_len, max_q, scale=None,
                           out=None, error=None, chunk_tokens=0, workspace=None):
    """q [T, Hq, d] bf16 (T = cu_q[-1], head dim d of 64 or 128); cu_q [B+1]
    int64; k_pool / v_pool [num_blocks, block_size, Hkv * d] bf16 (one layer's K
    and V sides of a PagedKVCache pool); block_table [B, max_blocks] int32;
    kv_len [B] int64 (keys per row, the new positions included); max_q >= every
    row's q_b. Returns out [T, Hq, d] bf16. Rows whose shape or pages are out of range are
    skipped and set `error` (an int32 [1] device tensor) when given. Each row's
    keys are split in chunks of `chunk_tokens` (0: the library's default) on
    separate workgroups; rows of several chunks merge fp32 partials held in
    `workspace` (a uint8 device tensor, allocated here when None); the chunks
    are launched longest first."""
    _lib.require_gpu(q, cu_q, k_pool, v_pool, block_table, kv_len)
    if q.dtype != torch.bfloat16 or k_pool.dtype != torch.bfloat16 or v_pool.dtype != torch.bfloat16:
        raise TypeError("verify_attention_paged: bf16 q and pools")
    T, hq, d = q.shape
    nb, bs, re = k_pool.shape
    if v_pool.shape != k_pool.shape or re % d != 0:
        raise ValueError("verify_attention_paged: k_pool / v_pool must be [num_blocks, bs, Hkv*d]")
    hkv = re // d
    B = cu_q.numel() - 1
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    if not (k_pool.is_contiguous() and v_pool.is_contiguous()):
        raise ValueError("verify_attention_paged: pools must be contiguous")
    q = q.contiguous()
    cu = cu_q.to(torch.int64).contiguous()
    kl = kv_len.to(torch.int64).contiguous()
    bt = block_table.to(torch.int32).contiguous()
    if out is None:
        out = torch.empty_like(q)
    if workspace is None:
        workspace = attention_workspace(B, max_q, hq, hkv, bs, bt.shape[1], chunk_tokens, q.device)
    rc = _lib.lib().sdx_verify_attention_paged(
        _lib.ptr(q), _lib.BF16, B, _lib.ptr(cu), int(max_q), hq, hkv, d,
        _lib.ptr(k_pool), _lib.ptr(v_pool), nb, bs, _lib.ptr(bt),
        bt.shape[1], _lib.ptr(kl), scale, int(chunk_tokens),
        _lib.ptr(workspace), workspace.numel(), _lib.ptr(out), _lib.ptr(error), _lib.stream_of(q))
    _lib.check(rc, "verify_attention_paged")
    return out

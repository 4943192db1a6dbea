"""The proposer-side device work of `vllm_draft_spec/proposer.py`, as HIP kernels.

The proposer's per-step arithmetic is a greedy draft token per request
(`logits.argmax(dim=-1)`, `proposer.py:262-263,331-332`) and the slot-mapping
bump for the next drafting step (`proposer.py:295-314`). Both are exposed here
so a vLLM-side integration (or this build's engine) calls the HIP kernels
instead of ATen's argmax / gather / masked_fill chain.
"""
import torch

from . import _lib

__all__ = ["greedy_draft_tokens", "drafting_slot_mapping", "PADDING_SLOT_ID"]

# vLLM's padding slot id (imported at proposer.py:47 from vllm's eagle.py); the
# value is a parameter of `drafting_slot_mapping`, this is its default.
PADDING_SLOT_ID = -1


def greedy_draft_tokens(logits):
    """argmax over the vocab (first index among maxima, -0 == +0). logits [..., V]."""
    _lib.require_gpu(logits)
    V = logits.shape[-1]
    x = logits.reshape(-1, V)
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        x = x.float()
    if not x.is_contiguous() or x.stride(-1) != 1:
        x = x.contiguous()
    out = torch.empty(x.shape[0], dtype=torch.int64, device=x.device)
    if x.shape[0]:
        rc = _lib.lib().sdx_argmax(_lib.ptr(x), _lib.dtype_code(x), x.shape[0], V, x.stride(0),
                                   _lib.ptr(out), _lib.stream_of(x))
        _lib.check(rc, "greedy_draft_tokens")
    return out.reshape(logits.shape[:-1])


def drafting_slot_mapping(block_table, positions, block_size, max_model_len,
                          padding_slot_id=PADDING_SLOT_ID):
    """Positions >= max_model_len are parked at 0 and get `padding_slot_id`;
    otherwise slot = block_table[r, pos // bs] * bs + pos % bs
    (`proposer.py:299-314`). Returns (clamped_positions, slot_mapping), int64."""
    _lib.require_gpu(block_table, positions)
    bt = block_table.to(torch.int32).contiguous()
    pos = positions.to(torch.int64).contiguous()
    rows = pos.numel()
    clamped = torch.empty(rows, dtype=torch.int64, device=pos.device)
    slots = torch.empty(rows, dtype=torch.int64, device=pos.device)
    if rows:
        rc = _lib.lib().sdx_slot_mapping(_lib.ptr(bt), rows, bt.shape[1], _lib.ptr(pos),
                                         int(block_size), int(max_model_len),
                                         int(padding_slot_id), _lib.ptr(clamped), _lib.ptr(slots),
                                         _lib.stream_of(pos))
        _lib.check(rc, "drafting_slot_mapping")
    return clamped, slots

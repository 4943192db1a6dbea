"""The reference's verify path as torch CPU ops: the CPU baseline of bench.py.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`): bench.py times it on the
host's cores beside the HIP path; nothing in the product imports it.

It follows the reference op for op, batched over rows as the engine does:
* `to_probs` (`specdec/sampling.py:34-67`): `logits.float()`, one-hot argmax
  for T <= 0, `softmax(logits / T)`, top-k zeroing without renormalisation,
  top-p by a descending sort, `cumsum`, `keep = cum - srt < top_p`,
  `keep[..., 0] = True`, scatter, then `probs / sum.clamp_min(1e-12)`;
* the accept block of `specdec/engine.py:281-312`: per position
  `ratio = p(x) / max(q(x), 1e-10)`, `ok = (u < min(ratio, 1)) & alive &
  (n_acc == i)`, `n_acc += ok`, `alive &= ok`; the stop position
  `min(n_acc, k - 1)`; the residual `clamp(p - q, 0)` normalised, or p when its
  mass is <= 1e-9 (`sampling.py:77-90`); the bonus row p_{k+1} when every
  draft was accepted.

Two choices differ from the literal reference, as in the HIP path and the
numpy oracle: the sort is stable (lower ids first among equal
probabilities), and the final draw is an inverse-CDF draw on the caller's
uniform (`torch.multinomial`'s noise stream cannot be reproduced). Its
probabilities come from torch's own softmax, so they agree with the oracle's
deterministic rule to rounding (about 1e-7), and its ids equal the oracle's
except where a decision sits within that rounding of flipping.
"""
import torch


def to_probs(logits, temperature=1.0, top_p=1.0, top_k=0):
    """`sampling.py:34-67` on torch CPU tensors [..., V] -> fp32 [..., V]."""
    logits = logits.float()
    V = logits.shape[-1]
    if temperature is None or temperature <= 0.0:                 # :43-48
        out = torch.zeros_like(logits)
        out.scatter_(-1, logits.argmax(dim=-1, keepdim=True), 1.0)
        return out
    probs = torch.softmax(logits / temperature, dim=-1)            # :50
    if top_k and 0 < top_k < V:                                    # :52-54
        kth = probs.topk(top_k, dim=-1).values[..., -1:]
        probs = torch.where(probs < kth, torch.zeros_like(probs), probs)
    if top_p is not None and 0.0 < top_p < 1.0:                    # :56-64
        srt, idx = torch.sort(probs, dim=-1, descending=True, stable=True)
        cum = srt.cumsum(dim=-1)
        keep = cum - srt < top_p
        keep[..., 0] = True
        mask = torch.zeros_like(probs, dtype=torch.bool).scatter_(-1, idx, keep)
        probs = torch.where(mask, probs, torch.zeros_like(probs))
    return probs / probs.sum(dim=-1, keepdim=True).clamp_min(1e-12)   # :66-67


def _draw(w, u):
    """Inverse-CDF draw per row of weights w [B, V] on uniforms u [B]: the first
    index whose float64 prefix sum exceeds u * total."""
    cdf = w.double().cumsum(dim=-1)
    t = (u.double() * cdf[:, -1]).unsqueeze(-1)
    return torch.searchsorted(cdf, t, right=True).squeeze(-1).clamp_max(w.shape[-1] - 1)


def rejection_sample(target_logits, draft_logits, draft_ids, u_accept, u_final,
                     temperature=1.0, top_p=1.0, top_k=0):
    """The verify step of `engine.py:281-312`: target [B, k+1, V], draft [B, k, V]
    logits (CPU tensors), draft_ids [B, k], u_accept [B, k], u_final [B].
    Returns (n_acc [B], y [B]) as int64 CPU tensors."""
    B, k1, _ = target_logits.shape
    k = k1 - 1
    p = [to_probs(target_logits[:, i], temperature, top_p, top_k) for i in range(k + 1)]
    q = [to_probs(draft_logits[:, i], temperature, top_p, top_k) for i in range(k)]
    ids = draft_ids.long()
    rows = torch.arange(B)
    n_acc = torch.zeros(B, dtype=torch.long)
    alive = torch.ones(B, dtype=torch.bool)
    for i in range(k):                                             # engine.py:285-295
        x = ids[:, i]
        ratio = p[i][rows, x] / q[i][rows, x].clamp_min(1e-10)
        ok = (u_accept[:, i] < ratio.clamp(max=1.0)) & alive & (n_acc == i)
        n_acc += ok.long()
        alive &= ok
    pick = n_acc.clamp(max=k - 1)                                  # engine.py:296-303
    p_stop = torch.stack(p[:k], dim=1)[rows, pick]
    q_stop = torch.stack(q, dim=1)[rows, pick]
    r = (p_stop - q_stop).clamp_min(0.0)                           # sampling.py:77-90
    tot = r.sum(dim=-1, keepdim=True)
    r = torch.where(tot <= 1e-9, p_stop, r)
    r = r / r.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    y_res = _draw(r, u_final)
    y_bonus = _draw(p[k], u_final)
    y = torch.where(n_acc == k, y_bonus, y_res)
    return n_acc, y

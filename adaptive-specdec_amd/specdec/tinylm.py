"""A one-layer decoder with seeded random weights, run on this build's paged KV
and verify-attention kernels: the stand-in model of the engine's tests and
bench (there are no checkpoints here).

forward(tokens [B, q], cache) appends the q new positions' K/V at the cache's
device lengths (`PagedKVCache.append`, the paged form of `kvcache.py:61-74`),
attends with `verify_attention_paged` (query j of row b sees slots
s <= lengths[b] + j, `kvcache.py:138-162`) and returns bf16 logits [B, q, V];
as in the reference engine (`engine.py:_forward` then `cache.advance(q)`), the
caller commits the lengths afterwards.

Every per-position product runs on a [B, D] matrix, and attention keeps a row's
keys in one chunk, so a row's logits at a position are the same bits whether
the position arrives alone (autoregressive decoding) or among the k + 1
positions of a verify forward.
"""
import torch

from .attention import attention_workspace, verify_attention_paged
from .kvcache import PagedKVCache

__all__ = ["TinyLM"]

HEAD = 128
CHUNK = 1024  # keys per attention chunk: contexts up to 1024 keys stay in one


class TinyLM:
    def __init__(self, vocab, hq=2, hkv=1, max_pos=1024, seed=0, device="cuda", base=None,
                 noise=0.0, scale=1.0):
        """Weights ~ N(0, 1/fan_in). With `base` (another TinyLM) the weights are
        base's plus noise * N(0, 1/fan_in): a draft that agrees with its target
        on most tokens. `scale` multiplies the logits."""
        self.V, self.hq, self.hkv, self.max_pos = int(vocab), int(hq), int(hkv), int(max_pos)
        self.dtype = torch.bfloat16  # of the logits
        self.writes_out = True       # forward(..., out=) writes logits into a caller view
        self.D = self.hq * HEAD
        self.device = torch.device(device)
        g = torch.Generator(device="cpu").manual_seed(int(seed))

        def w(*shape, fan):
            return torch.randn(shape, generator=g) / fan ** 0.5

        D, Vq, Vkv = self.D, self.hq * HEAD, self.hkv * HEAD
        shapes = {"emb": ((self.V, D), 1), "pos": ((self.max_pos, D), 1), "wq": ((D, Vq), D),
                  "wk": ((D, Vkv), D), "wv": ((D, Vkv), D), "wo": ((Vq, D), Vq),
                  "wlm": ((D, self.V), D)}
        self.p = {}
        for name, (shape, fan) in shapes.items():
            t = w(*shape, fan=fan)
            if base is not None:
                t = base.p[name].float().cpu() + noise * t
            self.p[name] = t.to(self.device, torch.bfloat16).contiguous()
        if base is None and scale != 1.0:
            self.p["wlm"] = (self.p["wlm"].float() * scale).to(torch.bfloat16).contiguous()
        self._ws = {}

    def new_cache(self, batch, capacity, block_size=16, seed=0):
        """A paged cache with room for `capacity` positions per row behind a shuffled
        block table."""
        mb = (int(capacity) + block_size - 1) // block_size
        c = PagedKVCache(1, batch, batch * mb, block_size, self.hkv, HEAD, mb,
                         dtype=torch.bfloat16, device=self.device)
        g = torch.Generator(device="cpu").manual_seed(int(seed))
        c.block_table.copy_(torch.randperm(batch * mb, generator=g).to(torch.int32).view(batch, mb))
        return c

    def forward(self, tokens, cache, out=None):
        """tokens [B, q] int64 (q <= 64 // (hq / hkv)) -> logits [B, q, V] bf16,
        written into `out` ([B, q, V], rows of unit stride) when given."""
        B, q = tokens.shape
        p = self.p
        pos = (cache.lengths.view(B, 1) + torch.arange(q, device=self.device).view(1, q))
        h = p["emb"][tokens] + p["pos"][pos.clamp(max=self.max_pos - 1)]          # [B, q, D]
        qs, ks, vs = [], [], []
        for j in range(q):
            hj = h[:, j].contiguous()
            qs.append(torch.mm(hj, p["wq"]))
            ks.append(torch.mm(hj, p["wk"]))
            vs.append(torch.mm(hj, p["wv"]))
        staged = torch.stack([torch.stack(ks, 1), torch.stack(vs, 1)]).unsqueeze(0)  # [1,2,B,q,Hkv*128]
        cache.append(staged)
        Q = torch.stack(qs, 1).reshape(B * q, self.hq, HEAD)
        cu_q = torch.arange(B + 1, device=self.device, dtype=torch.int64) * q
        kv_len = cache.lengths + q
        key = (B, q, cache.block_size, cache.max_blocks)
        if key not in self._ws:
            self._ws[key] = attention_workspace(B, q, self.hq, self.hkv, cache.block_size,
                                                cache.max_blocks, CHUNK, self.device)
        att = verify_attention_paged(Q, cu_q, cache.pool[0, 0], cache.pool[0, 1],
                                     cache.block_table, kv_len, q, chunk_tokens=CHUNK,
                                     workspace=self._ws[key]).view(B, q, self.D)
        logits = []
        for j in range(q):
            hj = h[:, j] + torch.mm(att[:, j].contiguous(), p["wo"])
            if out is not None:
                torch.mm(hj.contiguous(), p["wlm"], out=out[:, j])
            else:
                logits.append(torch.mm(hj.contiguous(), p["wlm"]))
        return out if out is not None else torch.stack(logits, 1)                  # [B, q, V]

    def prefill(self, prompt, cache, plen=None, chunk=16):
        """Right-padded prompt [B, P] with real lengths plen [B] (None: all P) ->
        logits at each row's last real position [B, V] (`engine.py:189-195`); the
        cache then holds each row's own prompt (lengths = plen). Attention is
        causal, so a real position never sees the pad after it, and the pad's K/V
        lie past the row's length, where the next forward overwrites them."""
        B, P = prompt.shape
        last = (torch.full((B,), P, dtype=torch.int64) if plen is None
                else torch.as_tensor(plen, dtype=torch.int64)).to(self.device) - 1
        out = torch.empty((B, self.V), dtype=self.dtype, device=self.device)
        for s in range(0, P, chunk):
            t = prompt[:, s:s + chunk].contiguous()
            logits = self.forward(t, cache)
            cache.commit(t.shape[1])
            here = (last >= s) & (last < s + t.shape[1])
            off = (last - s).clamp(0, t.shape[1] - 1)
            pick = logits[torch.arange(B, device=self.device), off]
            out = torch.where(here.view(B, 1), pick, out)
        cache.lengths.copy_(last + 1)
        return out

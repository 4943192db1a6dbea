"""A transformers causal LM as a `SpecEngine` model: the reference engine's own
model path (`specdec/engine.py:166-195`) over `RaggedCache`.

`forward(tokens, cache)` is `SpecDecodeEngine._forward` (`engine.py:172-183`):
positions from the cache's per-row lengths, the additive mask of
`kvcache.py:138-162` (built by this build's kernel), `past_key_values=cache`
(the K/V scatter is this build's kernel) and the cache's `cache_position`.
`prefill` is `_prefill` (`engine.py:189-195`): a right-padded prompt forward
with `valid = plen`, then `set_lengths(plen)` and the logits at each row's last
real token. The engine commits lengths with `cache.commit(q)` (the reference's
`advance`) and rolls them back on the device.

The forward's shapes follow the cache's host lengths, so rounds over this model
run eagerly (no graph capture); the engine refreshes the host lengths at its
one read per round.
"""
import torch

from .kvcache import RaggedCache

__all__ = ["HFCausalLM"]


class HFCausalLM:
    """Wrap a transformers causal LM (e.g. `Qwen3ForCausalLM`) for `SpecEngine`.

    logits_dtype: the dtype of the logits handed to the sampling kernels
    (default: the model's own dtype, e.g. float32 for a float32 model).
    """

    def __init__(self, model, logits_dtype=None):
        self.model = model.eval()
        cfg = model.config
        self.V = int(cfg.vocab_size)
        self.n_layers = int(cfg.num_hidden_layers)
        self.device = next(model.parameters()).device
        self.model_dtype = next(model.parameters()).dtype
        self.dtype = logits_dtype or self.model_dtype
        if self.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise TypeError(f"logits dtype {self.dtype} is not one the sampling kernels take")

    def new_cache(self, batch, capacity, seed=0):
        """A `RaggedCache` with room for `capacity` positions per row (`engine.py:166-168`)."""
        return RaggedCache(self.n_layers, batch, capacity, self.device)

    def forward(self, tokens, cache, valid=None):
        """tokens [B, q] -> logits [B, q, V] (`engine.py:172-183`); appends the
        positions' K/V at each row's length (the caller commits the lengths)."""
        q = tokens.shape[1]
        with torch.no_grad():
            out = self.model(input_ids=tokens, position_ids=cache.positions(q),
                             attention_mask=cache.attn_mask(q, self.model_dtype, valid=valid),
                             past_key_values=cache, cache_position=cache.cache_position(q),
                             use_cache=True)
        return out.logits.to(self.dtype)

    def prefill(self, prompt, cache, plen=None):
        """Right-padded prompt [B, P], real lengths plen [B] (None: P) -> logits at
        each row's last real token [B, V] (`engine.py:189-195`); the cache then
        holds each row's prompt alone."""
        B, P = prompt.shape
        pl = (torch.full((B,), P, dtype=torch.int64) if plen is None
              else torch.as_tensor(plen, dtype=torch.int64)).to(self.device)
        logits = self.forward(prompt, cache, valid=pl)
        cache.set_lengths(pl)                       # the pad is not part of the row
        idx = (pl - 1).view(-1, 1, 1).expand(-1, 1, logits.shape[-1])
        return logits.gather(1, idx).squeeze(1)

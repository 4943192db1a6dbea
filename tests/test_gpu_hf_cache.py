"""`RaggedCache` driven by a transformers model forward, on the GPU: the
invariants of the reference's `tests/test_kv_rollback.py:40-90` through this
build's scatter, mask and rollback kernels.

* a right-padded prefill (`valid` lengths) gives each row the logits of its
  own unpadded prompt;
* after speculating 4 tokens and rolling back to a different kept count per
  row, the next forward equals a cache that only ever saw the kept prefix;
* values written past a row's length are unreachable;
* the same with the sync-free `rollback_device` (the counts stay on the device).

The model is a tiny random Qwen3 (transformers' own implementation, fp32,
SDPA attention), the reference's test model shape; no checkpoint is loaded.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-4   # the reference test's threshold (fp32 logits)

transformers = pytest.importorskip("transformers")


def _model(seed=0, hidden=32, layers=2):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=16, hidden_size=hidden, intermediate_size=2 * hidden,
                      num_hidden_layers=layers, num_attention_heads=4, num_key_value_heads=2,
                      head_dim=8, max_position_embeddings=256, tie_word_embeddings=True)
    torch.manual_seed(seed)
    return Qwen3ForCausalLM(cfg).eval().to(DEV)


def _forward(m, cache, tokens, valid=None):
    q = tokens.shape[1]
    out = m(input_ids=tokens, position_ids=cache.positions(q),
            attention_mask=cache.attn_mask(q, torch.float32, valid=valid),
            past_key_values=cache, cache_position=cache.cache_position(q), use_cache=True)
    return out.logits


def _plain(m, seq):
    return m(input_ids=seq.unsqueeze(0), use_cache=True).logits[0, -1]


@pytest.fixture(scope="module")
def setup():
    from specdec.kvcache import RaggedCache
    m = _model()
    g = torch.Generator(device="cpu").manual_seed(0)
    B, P = 3, 7
    ids = torch.randint(0, 16, (B, P), generator=g).to(DEV)
    plen = torch.tensor([7, 5, 6])
    spec = torch.randint(0, 16, (B, 4), generator=g).to(DEV)
    keep = torch.tensor([4, 1, 2])
    nxt = torch.randint(0, 16, (B, 1), generator=g).to(DEV)
    return m, RaggedCache, ids, plen, spec, keep, nxt


@torch.inference_mode()
def test_padded_prefill_matches_unpadded_rows(setup):
    m, RaggedCache, ids, plen, _, _, _ = setup
    c = RaggedCache(m.config.num_hidden_layers, 3, 128, DEV)
    lg = _forward(m, c, ids, valid=plen)
    c.set_lengths(plen)
    for b in range(3):
        d = (lg[b, plen[b] - 1] - _plain(m, ids[b, :plen[b]])).abs().max().item()
        assert d < TOL, (b, d)
    assert int(c.error.item()) == 0


@pytest.mark.parametrize("device_rollback", [False, True])
@torch.inference_mode()
def test_rollback_equals_never_rolled_back(setup, device_rollback):
    m, RaggedCache, ids, plen, spec, keep, nxt = setup
    c = RaggedCache(m.config.num_hidden_layers, 3, 128, DEV)
    _forward(m, c, ids, valid=plen)
    c.set_lengths(plen)
    _forward(m, c, spec)
    c.advance(4)
    if device_rollback:
        c.rollback_device((4 - keep).to(DEV))        # no host sync
    else:
        c.rollback(4 - keep)
    got = _forward(m, c, nxt)
    assert c.lengths.cpu().tolist() == (plen + keep).tolist()
    for b in range(3):
        seq = torch.cat([ids[b, :plen[b]], spec[b, :keep[b]], nxt[b]])
        d = (got[b, -1] - _plain(m, seq)).abs().max().item()
        assert d < TOL, (b, d)
    # one more step on top, through advance (device lengths while the mirror is stale)
    c.advance(1)
    nxt2 = (nxt + 3) % 16
    got2 = _forward(m, c, nxt2)
    for b in range(3):
        seq = torch.cat([ids[b, :plen[b]], spec[b, :keep[b]], nxt[b], nxt2[b]])
        d = (got2[b, -1] - _plain(m, seq)).abs().max().item()
        assert d < TOL, (b, d)
    assert int(c.error.item()) == 0


@torch.inference_mode()
def test_stale_tail_is_unreachable(setup):
    m, RaggedCache, ids, plen, spec, keep, nxt = setup
    outs = []
    for corrupt in (False, True):
        c = RaggedCache(m.config.num_hidden_layers, 3, 128, DEV)
        _forward(m, c, ids, valid=plen)
        c.set_lengths(plen)
        _forward(m, c, spec)
        c.advance(4)
        c.rollback(4 - keep)
        if corrupt:
            lens = c.lengths.cpu().tolist()
            for layer in c.layers:
                for b in range(3):
                    layer.keys[b, :, lens[b]:, :] = 99.0
                    layer.values[b, :, lens[b]:, :] = 99.0
        outs.append(_forward(m, c, nxt).clone())
    assert (outs[0] - outs[1]).abs().max().item() < TOL

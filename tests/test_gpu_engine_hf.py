"""The speculative engine on the reference's own model path: tiny random Qwen3
models (transformers' implementation, fp32) over `RaggedCache`, driven by
`SpecEngine` through `specdec.hfmodel.HFCausalLM`.

* G2 as `tests/test_greedy_equivalence.py:32-82` states it: greedy speculative
  decoding emits the target's own greedy tokens at k = 1, 2, 3, 4, 6 and 8,
  under the EWMA controller with and without the confidence early exit, for a
  batch of one as for a batch of four, with a draft of another architecture,
  from right-padded prompts of different lengths; and the rejection path is
  taken (alpha < 0.99).
* G1 Part B as `tests/test_rejection_sampling.py:130-177` states it: B = 2048 x
  40 runs of the whole device round (draft steps, verify, round commit) at k =
  4, T = 1, top-p 0.9; the first token's distribution against the target's and
  the second token's against the exact autoregressive marginal, TV < 0.02.

The exact marginal uses the oracle's to_probs on the target's logits. No
checkpoint is loaded: the models are seeded random Qwen3 configurations of the
reference's test shape (vocab 16, 4 heads, 2 KV heads, head dim 8).
"""
import copy

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
VOCAB = 16
TV_GATE = 0.02

transformers = pytest.importorskip("transformers")


def _config(hidden=32, layers=2):
    from transformers import Qwen3Config
    return Qwen3Config(vocab_size=VOCAB, hidden_size=hidden, intermediate_size=2 * hidden,
                       num_hidden_layers=layers, num_attention_heads=4, num_key_value_heads=2,
                       head_dim=8, max_position_embeddings=256, tie_word_embeddings=True)


def _pair_arch():
    """Target 2 layers x hidden 32, draft 1 layer x hidden 16 (independent seeds)."""
    from transformers import Qwen3ForCausalLM
    torch.manual_seed(0)
    t = Qwen3ForCausalLM(_config(32, 2)).eval()
    torch.manual_seed(1)
    d = Qwen3ForCausalLM(_config(16, 1)).eval()
    return t.to(DEV), d.to(DEV)


def _pair_noisy(noise=4.0, seed=0):
    """Draft = a copy of the target with Gaussian noise on every weight (scaled by
    the weight's own spread): it agrees with the target only in part."""
    from transformers import Qwen3ForCausalLM
    torch.manual_seed(seed)
    t = Qwen3ForCausalLM(_config(32, 2)).eval()
    d = copy.deepcopy(t).eval()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for prm in d.parameters():
            prm.add_(torch.randn(prm.shape, generator=g) * noise * prm.std().clamp_min(1e-3))
    return t.to(DEV), d.to(DEV)


def _wrap(t, d):
    from specdec.hfmodel import HFCausalLM
    return HFCausalLM(t), HFCausalLM(d)


@pytest.fixture(scope="module")
def prompts():
    g = torch.Generator().manual_seed(0)
    B, P = 4, 6
    ids = torch.randint(0, VOCAB, (B, P), generator=g).to(DEV)
    plen = torch.tensor([P, P - 1, P - 2, P])      # ragged on purpose
    return ids, plen


@pytest.fixture(scope="module")
def noisy():
    return _wrap(*_pair_noisy(4.0))


NEW = 24


def _engine(tgt, drf, B, k, **kw):
    from specdec.engine import SpecEngine
    return SpecEngine(tgt, drf, B, k, temperature=0.0, max_new=NEW, prompt_len=8, device=DEV,
                      **kw)


def _ar(tgt, ids, plen):
    from specdec.engine import autoregressive
    return [o[:NEW] for o in autoregressive(tgt, ids, NEW, plen=plen)]


@pytest.mark.parametrize("k", [1, 2, 3, 4, 6, 8])
def test_hf_greedy_identical_to_autoregressive(noisy, prompts, k):
    tgt, drf = noisy
    ids, plen = prompts
    ar = _ar(tgt, ids, plen)
    print(f"[G2 hf] k={k} B={ids.shape[0]} plen={plen.tolist()}", flush=True)
    out = _engine(tgt, drf, ids.shape[0], k).generate(ids, plen)
    assert [o[:NEW] for o in out] == ar


@pytest.mark.parametrize("tau", [None, 0.5])
def test_hf_greedy_identical_under_controller(noisy, prompts, tau):
    """EWMA (`make_controller("ewma")`) and EWMA + early exit at tau 0.5."""
    from specdec.controller import DeviceController
    tgt, drf = noisy
    ids, plen = prompts
    B = ids.shape[0]
    ar = _ar(tgt, ids, plen)
    ctl = DeviceController(B, "batch", k_max=8, device=DEV)
    ks = []
    eng = _engine(tgt, drf, B, 8, controller=ctl, tau=tau)
    out = eng.generate(ids, plen, on_round=lambda e: ks.append(e.last_k))
    assert [o[:NEW] for o in out] == ar, f"k used {sorted(set(ks))}"
    # the observed draft / target cost ratio reached the controller (c moved from 0.15)
    assert ctl.host_state()[0][2] != 0.15


def test_hf_batch_of_one_agrees(noisy, prompts):
    tgt, drf = noisy
    ids, plen = prompts
    ar = _ar(tgt, ids, plen)
    out1 = _engine(tgt, drf, 1, 5).generate(ids[:1], plen[:1])
    assert out1[0][:NEW] == ar[0]


def test_hf_mismatched_draft_architecture():
    tgt, drf = _wrap(*_pair_arch())
    g = torch.Generator().manual_seed(0)
    ids = torch.randint(0, VOCAB, (4, 6), generator=g).to(DEV)
    plen = torch.tensor([6, 5, 4, 6])
    ar = _ar(tgt, ids, plen)
    out = _engine(tgt, drf, 4, 4).generate(ids, plen)
    assert [o[:NEW] for o in out] == ar


def test_hf_rejection_path_exercised(noisy, prompts):
    """Non-vacuity: at k = 8 the draft is rejected often enough (alpha < 0.99)."""
    tgt, drf = noisy
    ids, plen = prompts
    acc = [0, 0]   # accepted, positions reached (RunStats.alpha_conditional)

    def count(e):
        for a in e.n_acc.cpu().tolist():
            acc[0] += a
            acc[1] += min(a + 1, e.last_k)

    _engine(tgt, drf, ids.shape[0], 8).generate(ids, plen, on_round=count)
    alpha = acc[0] / max(1, acc[1])
    print(f"[G2 hf] alpha at k=8: {alpha:.3f}", flush=True)
    assert alpha < 0.99


def _tv(a, b):
    return 0.5 * float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).sum())


def _empirical(tokens):
    c = np.bincount(np.asarray(tokens, np.int64), minlength=VOCAB).astype(np.float64)
    return c / c.sum()


def test_g1_part_b_device_round_matches_exact_marginal():
    """`test_rejection_sampling.py:130-177` through this build's whole round."""
    from oracle import sampling as O
    from specdec.engine import SpecEngine
    t, d = _pair_arch()
    tgt, drf = _wrap(t, d)
    T, tp = 1.0, 0.9
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, VOCAB, (1, 5), generator=g).to(DEV)
    with torch.no_grad():
        lg = t(input_ids=prompt).logits[0, -1].float().cpu().numpy()
        p0 = O.to_probs(lg[None], T, tp)[0].astype(np.float64)
        marg = np.zeros(VOCAB)
        for t0 in range(VOCAB):
            if p0[t0] <= 0:
                continue
            seq = torch.cat([prompt[0], torch.tensor([t0], device=DEV)]).unsqueeze(0)
            l1 = t(input_ids=seq).logits[0, -1].float().cpu().numpy()
            marg += p0[t0] * O.to_probs(l1[None], T, tp)[0]
    B, REPS = 2048, 40
    ids = prompt.expand(B, -1).contiguous()
    eng = SpecEngine(tgt, drf, B, 4, temperature=T, top_p=tp, max_new=2, prompt_len=5, device=DEV)
    first, second, acc = [], [], [0, 0]

    def count(e):
        for a in e.n_acc.cpu().tolist():
            acc[0] += a
            acc[1] += min(a + 1, e.last_k)

    for r in range(REPS):
        out = eng.generate(ids, seed=1000 + r, on_round=count)
        first += [o[0] for o in out]
        second += [o[1] for o in out]
    d0 = _tv(_empirical(first), p0)
    d1 = _tv(_empirical(second), marg)
    alpha = acc[0] / max(1, acc[1])
    print(f"[G1 B] N={len(second)} alpha={alpha:.3f} TV0={d0:.4f} TV1={d1:.4f}", flush=True)
    assert 0.05 < alpha < 0.99          # both accept and reject paths taken
    assert d0 < TV_GATE, d0              # control: token 0 comes from the target alone
    assert d1 < TV_GATE, d1

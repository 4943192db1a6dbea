"""GPU parity of the device-side round: the fused draft step, the round commit,
the on-device controller and the engine built on them.

* draft step vs `oracle.sampling.draft_step`: ids, q(x) and conf bit for bit,
  the early-exit flag exactly (including its comparison direction at the tie);
* round commit vs `oracle.engine.round_commit`: emitted tokens, lengths, done
  flags and cache rollback, fixed and per-row k;
* controller vs `oracle.controller.EWMAState`: k exactly, state to 1e-12;
* the engine: greedy output identical to target-only decoding (the reference's
  G2 gate, `tests/test_engine.py`), sampled rounds checked round by round
  against the oracle on the models' own logits, graph replays identical to
  eager rounds, the early exit and the controller inside the loop.
"""
import numpy as np
import pytest
import torch

from oracle import controller as OC
from oracle import engine as OE
from oracle import sampling as O
from specdec import _lib
from specdec.controller import DeviceController
from specdec.engine import SpecEngine, autoregressive
from specdec.sampling import draft_step
from specdec.tinylm import TinyLM
from specdec.workloads import uniforms, zipf_logits

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().float().cpu().numpy()


def _bits_equal(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and bool(np.all(a.view(np.uint32) == b.view(np.uint32)))


# ------------------------------------------------------------------ draft step
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("T,tp,tk", [(1.0, 1.0, 0), (0.8, 0.95, 0), (0.7, 0.9, 50), (0.0, 1.0, 0)])
@pytest.mark.parametrize("B,V", [(1, 1000), (7, 4096), (64, 32000), (3, 151936)])
def test_draft_step_matches_oracle(dtype, T, tp, tk, B, V):
    g = torch.Generator(device=DEV).manual_seed(B * 7 + V)
    x = zipf_logits(B, V, g, DEV, dtype=dtype)
    u = uniforms((B,), g, DEV)
    conf0 = 0.3 + 0.7 * uniforms((B,), g, DEV)
    conf = conf0.clone()
    xs, qx, stop = draft_step(x, u, T, tp, tk, conf=conf, tau=0.5, step=2, min_k=1)
    rx, rq, rconf, rstop = O.draft_step(_np(x), _np(u), T, tp, tk, conf=_np(conf0), tau=0.5,
                                        step=2, min_k=1)
    torch.cuda.synchronize()
    assert np.array_equal(xs.cpu().numpy(), rx)
    assert _bits_equal(qx.cpu().numpy(), rq)
    assert _bits_equal(conf.cpu().numpy(), rconf)
    assert int(stop.item()) == rstop


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_draft_step_stop_rule(dtype):
    """mean(conf) < tau with the mean a row-order fp32 sum over B: tau equal to
    the mean does not stop, the next float up does; step < min_k never stops."""
    B, V = 7, 4096
    g = torch.Generator(device=DEV).manual_seed(5)
    x = zipf_logits(B, V, g, DEV, dtype=dtype)
    u = uniforms((B,), g, DEV)
    conf0 = 0.2 + 0.8 * uniforms((B,), g, DEV)
    _, _, rconf, _ = O.draft_step(_np(x), _np(u), 0.9, 1.0, 0, conf=_np(conf0), tau=0.5)
    s = np.float32(0.0)
    for v in rconf:
        s = np.float32(s + v)
    mean = np.float32(s / np.float32(B))
    cases = [(float(mean), 3, 1, 0), (float(np.nextafter(mean, np.float32(1))), 3, 1, 1),
             (float(np.nextafter(mean, np.float32(1))), 2, 3, 0)]
    for tau, step, min_k, want in cases:
        c = conf0.clone()
        _, _, stop = draft_step(x, u, 0.9, 1.0, 0, conf=c, tau=tau, step=step, min_k=min_k)
        assert int(stop.item()) == want, (tau, step, min_k)
        assert _bits_equal(c.cpu().numpy(), rconf)


def test_draft_step_without_conf_and_strided_rows():
    """No conf / tau (the plain fused step), rows read from a [B, 2, V] view."""
    B, V = 5, 2048
    g = torch.Generator(device=DEV).manual_seed(9)
    full = zipf_logits(B * 2, V, g, DEV).view(B, 2, V)
    x = full[:, 1]
    u = uniforms((B,), g, DEV)
    xs, qx, stop = draft_step(x, u, 0.8, 0.9, 0)
    rx, rq, _, _ = O.draft_step(_np(x), _np(u), 0.8, 0.9, 0)
    assert stop is None
    assert np.array_equal(xs.cpu().numpy(), rx)
    assert _bits_equal(qx.cpu().numpy(), rq)


# ------------------------------------------------------------------ round commit
def _commit_case(B, k, seed, ragged):
    rng = np.random.default_rng(seed)
    max_new = 10
    eos = [3, 7]
    if ragged:
        kb = rng.integers(0, 7, B)
        cu = np.concatenate([[0], np.cumsum(kb)]).astype(np.int64)
        n_acc = np.array([rng.integers(0, kb[b] + 1) for b in range(B)], np.int64)
        ids = rng.integers(0, 40, int(cu[-1])).astype(np.int64)
    else:
        cu = None
        n_acc = rng.integers(0, k + 1, B).astype(np.int64)
        ids = rng.integers(0, 40, (B, k)).astype(np.int64)
    y = rng.integers(0, 40, B).astype(np.int64)
    done = rng.random(B) < 0.2
    out_len = rng.integers(1, max_new, B).astype(np.int64)
    out = rng.integers(100, 200, (B, max_new)).astype(np.int64)
    len0 = rng.integers(16, 64, B).astype(np.int64)
    len1 = len0 + rng.integers(0, 3, B)
    return dict(max_new=max_new, eos=eos, cu=cu, n_acc=n_acc, ids=ids, y=y, done=done,
                out_len=out_len, out=out, len0=len0, len1=len1)


@pytest.mark.parametrize("ragged", [False, True])
@pytest.mark.parametrize("B", [1, 64, 300])
def test_round_commit_matches_oracle(B, ragged):
    k = 4
    c = _commit_case(B, k, B + 17 * ragged, ragged)
    d = {n: torch.from_numpy(np.ascontiguousarray(c[n])).to(DEV)
         for n in ("n_acc", "ids", "y", "out_len", "out", "len0", "len1")}
    done = torch.from_numpy(c["done"].astype(np.uint8)).to(DEV)
    cu = None if c["cu"] is None else torch.from_numpy(c["cu"]).to(DEV)
    eos = torch.tensor(c["eos"], dtype=torch.int64, device=DEV)
    pending = torch.full((B,), -5, dtype=torch.int64, device=DEV)
    rc = _lib.lib().sdx_round_commit(
        B, k, _lib.ptr(cu), _lib.ptr(d["n_acc"]), _lib.ptr(d["y"]), _lib.ptr(d["ids"]),
        _lib.ptr(done), _lib.ptr(d["out"]), _lib.ptr(d["out_len"]), c["max_new"], _lib.ptr(eos),
        len(c["eos"]), _lib.ptr(d["len0"]), _lib.ptr(d["len1"]), _lib.ptr(pending), None, None,
        _lib.stream_of(pending))
    _lib.check(rc, "sdx_round_commit")
    outs = [list(c["out"][b, :c["out_len"][b]]) for b in range(B)]
    drop, rdone, routs = OE.round_commit(c["n_acc"], c["y"], c["ids"], k, c["done"], outs,
                                         c["eos"], c["max_new"], cu_k=c["cu"])
    got_len = d["out_len"].cpu().numpy()
    got_out = d["out"].cpu().numpy()
    got_done = done.cpu().numpy().astype(bool)
    assert np.array_equal(got_done, rdone)
    for b in range(B):
        if c["done"][b]:        # a finished row is left as it was
            assert got_len[b] == c["out_len"][b]
            assert np.array_equal(got_out[b], c["out"][b])
            continue
        assert got_len[b] == len(routs[b]), b
        assert got_out[b, :got_len[b]].tolist() == routs[b], b
        assert np.array_equal(got_out[b, got_len[b]:], c["out"][b, got_len[b]:])
    assert np.array_equal(d["len0"].cpu().numpy(), c["len0"] - drop)
    assert np.array_equal(d["len1"].cpu().numpy(), c["len1"] - drop)
    assert np.array_equal(pending.cpu().numpy(), c["y"])


def test_round_commit_flags_raise_error_word():
    """A live row flagged NONFINITE / UNSUPPORTED / BAD_ROW / WORKSPACE, or with
    y < 0, emits nothing and is set done with pending 0, and the error word gets
    1 (flag) or 2 (y < 0); informational flags (near tie, tie order) and finished
    rows change nothing."""
    B, k, max_new = 8, 2, 10
    n_acc = torch.tensor([1, 1, 1, 1, 1, 1, 1, 1], dtype=torch.int64, device=DEV)
    y = torch.tensor([5, 6, 7, -1, 9, 10, 11, -1], dtype=torch.int64, device=DEV)
    ids = torch.arange(100, 100 + B * k, dtype=torch.int64, device=DEV)
    flags = torch.tensor([0, 2, 1 | 32, 0, 16, 8, 4, 2], dtype=torch.uint8, device=DEV)
    done = torch.tensor([0, 0, 0, 0, 0, 0, 0, 1], dtype=torch.uint8, device=DEV)
    out = torch.zeros((B, max_new), dtype=torch.int64, device=DEV)
    out_len = torch.ones(B, dtype=torch.int64, device=DEV)
    pending = torch.full((B,), -5, dtype=torch.int64, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    rc = _lib.lib().sdx_round_commit(
        B, k, None, _lib.ptr(n_acc), _lib.ptr(y), _lib.ptr(ids), _lib.ptr(done), _lib.ptr(out),
        _lib.ptr(out_len), max_new, None, 0, None, None, _lib.ptr(pending), _lib.ptr(flags),
        _lib.ptr(err), _lib.stream_of(pending))
    _lib.check(rc, "sdx_round_commit")
    assert int(err.item()) == 3
    assert out_len.cpu().tolist() == [3, 1, 3, 1, 1, 1, 1, 1]
    assert done.cpu().tolist() == [0, 1, 0, 1, 1, 1, 1, 1]
    assert pending.cpu().tolist() == [5, 0, 7, 0, 0, 0, 0, -1]
    assert out[0, 1:3].cpu().tolist() == [100, 5] and out[2, 1:3].cpu().tolist() == [104, 7]


# ------------------------------------------------------------------ controller
def test_controller_batch_matches_oracle():
    B, rounds = 16, 30
    rng = np.random.default_rng(3)
    dc = DeviceController(B, "batch", k_max=8, beta=0.99, k_init=4, c_init=0.15, warmup=3)
    oc = OC.EWMAState(k_max=8, beta=0.99, k_init=4, c_init=0.15, warmup=3)
    c_obs = torch.zeros(1, dtype=torch.float32, device=DEV)
    alpha = 0.8
    for r in range(rounds):
        k = oc.propose_k()
        assert int(dc.k[0]) == k, r
        if r == 12:
            alpha = 0.3          # the acceptance drops: k must follow
        n = np.minimum(rng.geometric(1 - alpha, B) - 1, k).astype(np.int64)
        cobs = None
        if r % 5 == 4:
            c_obs.fill_(0.05 + 0.02 * r)
            cobs = float(np.float32(0.05 + 0.02 * r))
        dc.update(torch.from_numpy(n).to(DEV), c_obs=c_obs if cobs is not None else None)
        oc.update(k, n, c_obs=cobs)
    oc.propose_k()
    acc, reached, c, nr, last_k = dc.host_state()[0]
    assert nr == oc.rounds and last_k == oc.last_k == int(dc.k[0])
    assert abs(acc - oc.acc) <= 1e-12 * max(1.0, abs(oc.acc))
    assert abs(reached - oc.reached) <= 1e-12 * max(1.0, abs(oc.reached))
    assert abs(c - oc.c) <= 1e-15


def test_controller_per_row_matches_oracle():
    B, rounds = 300, 12
    rng = np.random.default_rng(4)
    dc = DeviceController(B, "row", k_max=8, beta=0.95, k_init=3, c_init=0.1, warmup=2)
    ocs = [OC.EWMAState(k_max=8, beta=0.95, k_init=3, c_init=0.1, warmup=2) for _ in range(B)]
    alphas = rng.uniform(0.2, 0.95, B)
    for r in range(rounds):
        ks = np.array([o.propose_k() for o in ocs], np.int64)
        assert np.array_equal(dc.k.cpu().numpy(), ks), r
        assert np.array_equal(dc.cu_k.cpu().numpy(), np.concatenate([[0], np.cumsum(ks)])), r
        n = np.minimum(rng.geometric(1 - alphas) - 1, ks).astype(np.int64)
        dc.update(torch.from_numpy(n).to(DEV))
        for b in range(B):
            ocs[b].update(int(ks[b]), [int(n[b])])
    ks = np.array([o.propose_k() for o in ocs], np.int64)
    assert np.array_equal(dc.k.cpu().numpy(), ks)
    assert np.array_equal(dc.cu_k.cpu().numpy(), np.concatenate([[0], np.cumsum(ks)]))
    st = dc.host_state()
    for b in range(B):
        assert abs(st[b][0] - ocs[b].acc) <= 1e-12 * max(1.0, ocs[b].acc)
        assert abs(st[b][1] - ocs[b].reached) <= 1e-12 * max(1.0, ocs[b].reached)


# ------------------------------------------------------------------ engine
V_LM = 4096


@pytest.fixture(scope="module")
def models():
    tgt = TinyLM(V_LM, hq=2, hkv=1, seed=1, device=DEV, scale=4.0)
    drf = TinyLM(V_LM, hq=2, hkv=1, seed=2, device=DEV, base=tgt, noise=0.6)
    return tgt, drf


def _prompt(B, P, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randint(0, V_LM, (B, P), generator=g).to(DEV)


def test_tinylm_forward_matches_dense_reference(models):
    """The stand-in model on the paged cache vs the same maths in fp32 over
    dense K/V (causal over all positions), within bf16 rounding."""
    tgt, _ = models
    B, P = 3, 21
    prompt = _prompt(B, P, 11)
    cache = tgt.new_cache(B, 64)
    first = tgt.forward(prompt[:, :16], cache)
    cache.commit(16)
    got = torch.cat([first, tgt.forward(prompt[:, 16:], cache)], 1).float()
    p = {n: w.float() for n, w in tgt.p.items()}
    h = p["emb"][prompt] + p["pos"][torch.arange(P, device=DEV)]
    q = (h @ p["wq"]).view(B, P, 2, 128)
    kk = (h @ p["wk"]).view(B, P, 1, 128)
    vv = (h @ p["wv"]).view(B, P, 1, 128)
    s = torch.einsum("bqhd,bkd->bhqk", q, kk[:, :, 0].contiguous()) / 128 ** 0.5
    mask = torch.ones(P, P, device=DEV, dtype=torch.bool).tril()
    s = s.masked_fill(~mask, float("-inf")).softmax(-1)
    att = torch.einsum("bhqk,bkd->bqhd", s, vv[:, :, 0].contiguous()).reshape(B, P, 256)
    ref = (h + att @ p["wo"]) @ p["wlm"]
    err = (got - ref).abs().max().item()
    assert err < 0.05 * ref.abs().max().item(), err


@pytest.mark.parametrize("k", [1, 4])
@pytest.mark.parametrize("graphs", [False, True])
def test_engine_greedy_equals_autoregressive(models, k, graphs):
    """G2: at T = 0 speculative decoding emits exactly the target's own greedy
    sequence, whatever the draft proposes."""
    tgt, drf = models
    B, P, max_new = 5, 12, 40
    prompt = _prompt(B, P, 3)
    ref = autoregressive(tgt, prompt, max_new)
    eos = [ref[0][9], ref[2][20]]            # rows stop early at these tokens
    ref = autoregressive(tgt, prompt, max_new, eos_ids=eos)
    acc = []
    eng = SpecEngine(tgt, drf, B, k, temperature=0.0, eos_ids=eos, max_new=max_new,
                     prompt_len=P, device=DEV)
    got = eng.generate(prompt, graphs=graphs, on_round=lambda e: acc.append(e.n_acc.cpu()))
    assert got == ref
    assert int(eng.tcache.error.item()) == 0 and int(eng.dcache.error.item()) == 0
    mean_acc = torch.stack(acc).float().mean().item()
    assert 0.0 < mean_acc < k or k == 1      # the draft agrees only in part
    assert len(acc) < max_new                # speculation saved target forwards


def test_engine_sampled_rounds_match_oracle(models):
    """Each round of a sampled run, on the models' own logits: the drafted ids
    (fused draft step), n_acc and y (verify) and the emitted tokens, lengths
    and done flags (round commit) equal the oracle's."""
    tgt, drf = models
    B, P, k, max_new = 4, 10, 3, 24
    T, tp, tk = 0.8, 0.95, 0
    prompt = _prompt(B, P, 5)
    eng = SpecEngine(tgt, drf, B, k, temperature=T, top_p=tp, top_k=tk, max_new=max_new,
                     prompt_len=P, device=DEV)
    state = {}

    def check(e):
        if not state:   # after the first round: take the oracle's state from start()
            state["outs"] = [[int(t)] for t in state_first]
            state["done"] = np.zeros(B, bool)
            state["tlen"] = np.full(B, P, np.int64)
        dlog = _np(e.dlog)
        xs = e.xs.cpu().numpy()
        ud = _np(e.u_draft)
        for i in range(k):
            rx, _, _, _ = O.draft_step(dlog[:, i], ud[i], T, tp, tk)
            assert np.array_equal(xs[:, i], rx), (e.rounds, i)
        rn, ry, _ = O.rejection_sample(_np(e.last_target_logits), dlog, xs, _np(e.u_acc),
                                       _np(e.u_fin), T, tp, tk, active=~state["done"])
        assert np.array_equal(e.n_acc.cpu().numpy(), rn), e.rounds
        assert np.array_equal(e.y.cpu().numpy(), ry), e.rounds
        drop, state["done"], state["outs"] = OE.round_commit(rn, ry, xs, k, state["done"],
                                                            state["outs"], [], max_new)
        state["tlen"] = state["tlen"] + k + 1 - drop
        assert np.array_equal(e.tcache.lengths.cpu().numpy(), state["tlen"])
        assert np.array_equal(e.dcache.lengths.cpu().numpy(), state["tlen"])
        assert np.array_equal(e.done.cpu().numpy().astype(bool), state["done"])
        assert e.outputs() == state["outs"]

    # the first token (start) from the same generator stream as generate() uses
    g = torch.Generator(device=DEV).manual_seed(0)
    u_first = torch.rand(B, generator=g, device=DEV)
    tl = tgt.prefill(prompt, tgt.new_cache(B, 64))
    state_first, _, _, _ = O.draft_step(_np(tl), _np(u_first), T, tp, tk)
    out = eng.generate(prompt, seed=0, on_round=check)
    assert out == state["outs"]
    assert all(len(o) == max_new for o in out)


def test_engine_graph_replay_matches_eager(models):
    """Sampled decoding with every round replayed from a HIP graph emits the
    same tokens, round by round, as eager rounds on the same uniforms."""
    tgt, drf = models
    B, P, k, max_new = 6, 9, 4, 32
    prompt = _prompt(B, P, 8)
    runs = []
    for graphs in (False, True):
        eng = SpecEngine(tgt, drf, B, k, temperature=0.7, top_p=0.9, top_k=40, max_new=max_new,
                         eos_ids=[17], prompt_len=P, device=DEV)
        hist = []
        out = eng.generate(prompt, seed=21, graphs=graphs,
                           on_round=lambda e: hist.append((e.n_acc.cpu(), e.y.cpu())))
        runs.append((out, hist))
    (o0, h0), (o1, h1) = runs
    assert o0 == o1
    assert len(h0) == len(h1) and len(h0) > 2
    for (n0, y0), (n1, y1) in zip(h0, h1):
        assert torch.equal(n0, n1) and torch.equal(y0, y1)


def test_engine_early_exit_matches_oracle(models):
    """ConfidenceEarlyExit: a round stops drafting at the first step >= min_k
    where mean(conf) < tau; the verify then runs at that k."""
    tgt, drf = models
    B, P, k, max_new = 4, 8, 6, 20
    T, tau, min_k = 1.0, 0.05, 2
    prompt = _prompt(B, P, 13)
    eng = SpecEngine(tgt, drf, B, k, temperature=T, max_new=max_new, prompt_len=P, device=DEV,
                     tau=tau, min_k=min_k)
    seen = []

    def check(e):
        ke = e.last_k
        dlog = _np(e.dlog)
        ud = _np(e.u_draft)
        conf = np.ones(B, np.float32)
        want = k
        for i in range(k):
            _, _, conf, stop = O.draft_step(dlog[:, i], ud[i], T, conf=conf, tau=tau,
                                            step=i + 1, min_k=min_k)
            if stop and i + 1 < k:
                want = i + 1
                break
        assert ke == want
        xs = e.xs[:, :ke].cpu().numpy()
        done_before = seen[-1][2] if seen else np.zeros(B, bool)
        rn, ry, _ = O.rejection_sample(_np(e.last_target_logits), dlog[:, :ke], xs,
                                       _np(e.u_acc)[:, :ke], _np(e.u_fin), T,
                                       active=~done_before)
        assert np.array_equal(e.n_acc.cpu().numpy(), rn)
        assert np.array_equal(e.y.cpu().numpy(), ry)
        seen.append((ke, rn, e.done.cpu().numpy().astype(bool)))

    eng.generate(prompt, seed=4, on_round=check)
    assert any(s[0] < k for s in seen), "tau never cut a round short"


@pytest.mark.parametrize("graphs", [False, True])
def test_engine_device_controller(models, graphs):
    """The batch controller inside the loop: each round's k equals the oracle
    controller's proposal given the rounds' n_acc; with graphs one graph per k."""
    tgt, drf = models
    B, P, kmax, max_new = 4, 8, 6, 40
    prompt = _prompt(B, P, 17)
    ctl = DeviceController(B, "batch", k_max=kmax, beta=0.98, k_init=3, warmup=2, device=DEV)
    oc = OC.EWMAState(k_max=kmax, beta=0.98, k_init=3, warmup=2)
    eng = SpecEngine(tgt, drf, B, kmax, temperature=0.0, max_new=max_new, prompt_len=P,
                     device=DEV, controller=ctl, observe_cost=False)
    ks = []

    def check(e):
        k = oc.propose_k()
        assert e.last_k == k
        oc.update(k, e.n_acc.cpu().numpy())
        ks.append(k)

    out = eng.generate(prompt, graphs=graphs, on_round=check)
    assert out == autoregressive(tgt, prompt, max_new)
    assert oc.propose_k() == int(ctl.k[0])
    assert len(ks) > 3


@pytest.mark.parametrize("graphs", [False, True])
def test_engine_ragged_prompts_greedy(models, graphs):
    """Right-padded prompts with per-row lengths (`engine.py:189-226`): each row
    decodes as it would alone from its unpadded prompt, and greedy speculative
    decoding still equals target-only decoding from the same padded batch."""
    tgt, drf = models
    B, P, max_new = 4, 12, 30
    prompt = _prompt(B, P, 23)
    plen = torch.tensor([12, 7, 9, 1])
    ref = autoregressive(tgt, prompt, max_new, plen=plen)
    for b in range(B):   # a row alone, unpadded, gives the same tokens
        alone = autoregressive(tgt, prompt[b:b + 1, :int(plen[b])].contiguous(), max_new)
        assert alone[0] == ref[b], b
    eng = SpecEngine(tgt, drf, B, 3, temperature=0.0, max_new=max_new, prompt_len=P, device=DEV)
    assert eng.generate(prompt, plen, graphs=graphs) == ref
    assert eng.tcache.lengths.tolist() == eng.dcache.lengths.tolist()


def test_engine_rejects_prompt_past_capacity(models):
    tgt, drf = models
    eng = SpecEngine(tgt, drf, 2, 4, temperature=0.0, max_new=8, capacity=20, device=DEV)
    with pytest.raises(ValueError, match="capacity"):
        eng.start(_prompt(2, 9, 1))
    eng.start(_prompt(2, 7, 1))        # 7 + 8 + 4 + 1 = 20 fits


def test_engine_raises_on_flagged_rows(models):
    """A target whose logits hold +inf: the verify flags the rows NONFINITE, the
    round commit emits nothing for them and raises its error word, and the
    engine's next read raises instead of emitting tokens."""
    tgt, drf = models

    class InfLM(TinyLM):
        def forward(self, tokens, cache):
            out = super().forward(tokens, cache)
            out[..., 7] = float("inf")
            return out

    bad = InfLM(V_LM, hq=2, hkv=1, seed=1, device=DEV, scale=4.0)
    eng = SpecEngine(bad, drf, 3, 2, temperature=0.8, top_p=0.9, max_new=10, prompt_len=6,
                     device=DEV)
    with pytest.raises(RuntimeError, match="NONFINITE|no token"):
        eng.generate(_prompt(3, 6, 2), seed=1)
    assert eng.out_len.cpu().tolist() == [1, 1, 1]   # only the first token went out

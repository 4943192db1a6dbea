"""A speculative-decoding round with its bookkeeping on the device.

The counterpart of the reference's `SpecDecodeEngine.generate` round
(`specdec/engine.py:228-342`):
  1. up to k draft forwards, each followed by one fused draft step (to_probs,
     the draw, conf *= q(x): `engine.py:246-258`), then the commit-only forward;
  2. one target forward over [pending, x_1..x_k] (`engine.py:266-275`);
  3. the accept test and residual / bonus draw in one call (`engine.py:281-303`);
  4. the end of the round in one kernel: rollback of both caches by k - n_acc,
     emission with the EOS / max_new stops, pending = y (`engine.py:305-340`),
     where the reference syncs the host (`n_acc.tolist()`) and loops in Python;
  5. the controller's update on the device (`controller.py:143-154`).
Nothing in a round at a fixed k waits for the host, so such a round is captured
in one HIP graph per k (`SpecEngine.capture`) and replayed. The host reads the
device only where the reference's control flow needs a value: the loop
condition (`all_done`, `engine.py:232`), the controller's k for the next round
and the early-exit decision (`controller.py:184-187`, one read per draft step,
as the reference's `float(conf.mean())`), and `outputs()`.

Models follow `specdec.tinylm.TinyLM` (paged cache, graph-capturable) or
`specdec.hfmodel.HFCausalLM` (a transformers causal LM over `RaggedCache`, the
reference's own model path, `engine.py:166-183`): `forward(tokens [B, q], cache)`
returns logits [B, q, V] (of the model's `dtype`) and appends the positions' K/V
at the cache's device lengths; `prefill(prompt, cache, plen)` takes right-padded
prompts with per-row lengths and leaves each row's cache at its own length
(`engine.py:189-195`); the engine commits the lengths (`cache.commit(q)`,
`kvcache.py:165-168`). Every draw takes the caller's uniforms from static
buffers (u_draft [k, B], u_acc [B, k], u_fin [B]) filled before each round;
`generate` fills them from one device generator.

The one host read per round (`sync`, where the reference reads `n_acc.tolist()`)
also brings back an error word: the round commit raises it for a live row the
verify flagged (NONFINITE / UNSUPPORTED / BAD_ROW / WORKSPACE) or left without
a token, and the caches' kernels raise theirs on overflow or a rollback below
zero. `sync` raises `RuntimeError` then, as the reference fails loudly there
(torch.multinomial on NaN probabilities). Caches that keep host lengths
(`RaggedCache`) get them from the same read.

Differences from the reference, by design: a row stops at max_new tokens also
when max_new is 1 (the reference's first token ignores the limit); one uniform
u_fin serves the residual or the bonus draw, whichever the row takes; the
controller's observed cost ratio c_obs (draft over target forward time,
`engine.py:344-346`) comes from device event timings of the eager rounds,
reaches the controller one round later than in the reference, and keeps its
last value while rounds replay from graphs.
"""
import torch

from . import _lib
from .sampling import Verifier, _switch_args, draft_step

__all__ = ["SpecEngine", "autoregressive"]


class SpecEngine:
    """Speculative decoding of a batch with a target and a draft model.

    k is the largest draft length (buffers are sized for it); a round drafts
    k_round <= k tokens. controller: a `specdec.controller.DeviceController`
    in batch mode (its device k picks each round's length) or None (always k).
    tau / min_k: the confidence early exit of `ConfidenceEarlyExit`
    (`controller.py:162-191`), or tau None for none.
    """

    def __init__(self, target, draft, batch, k, temperature=0.0, top_p=1.0, top_k=0,
                 eos_ids=(), max_new=64, capacity=None, prompt_len=0, device="cuda", seed=0,
                 controller=None, tau=None, min_k=1, observe_cost=True):
        if controller is not None and getattr(controller, "mode", "batch") != "batch":
            raise ValueError("SpecEngine drafts one k per round: use a batch-mode controller")
        self.target, self.draft = target, draft
        self.B, self.k = int(batch), int(k)
        if self.k < 1:
            raise ValueError("k must be >= 1")
        self.V = target.V
        if draft.V != self.V:
            raise ValueError(f"target vocab {self.V} != draft vocab {draft.V}; speculative "
                             "decoding requires a shared tokenizer")
        self.dtype = getattr(target, "dtype", torch.bfloat16)
        if getattr(draft, "dtype", torch.bfloat16) != self.dtype:
            raise ValueError("target and draft logits must share a dtype")
        self.temperature, self.top_p, self.top_k = temperature, top_p, top_k
        self.T, self.tp, self.tk = _switch_args(temperature, top_p, top_k)
        self.max_new = int(max_new)
        self.tau = None if tau is None else float(tau)
        self.min_k = int(min_k)
        dev = torch.device(device)
        self.device = dev
        cap = capacity or (int(prompt_len) + 2 * self.max_new + self.k + 2)
        self.capacity = int(cap)
        self.tcache = target.new_cache(self.B, cap, seed=seed)
        self.dcache = draft.new_cache(self.B, cap, seed=seed + 1)
        B, k, V = self.B, self.k, self.V
        # error words: the round commit's, then the two caches' (their kernels write
        # through these views), read back with `done` in one copy per round
        self.err = torch.zeros(3, dtype=torch.int32, device=device)
        self.tcache.error = self.err[1:2]
        self.dcache.error = self.err[2:3]
        eos = [int(e) for e in eos_ids]
        self.eos = torch.tensor(eos or [-1], dtype=torch.int64, device=dev)
        self.n_eos = len(eos)
        self.pending = torch.zeros(B, dtype=torch.int64, device=dev)
        self.done = torch.zeros(B, dtype=torch.uint8, device=dev)
        self.active = torch.ones(B, dtype=torch.uint8, device=dev)
        self.out = torch.zeros((B, self.max_new), dtype=torch.int64, device=dev)
        self.out_len = torch.zeros(B, dtype=torch.int64, device=dev)
        self.xs = torch.zeros((B, k), dtype=torch.int64, device=dev)
        self.dlog = torch.zeros((B, k, V), dtype=self.dtype, device=dev)
        self.vin = torch.zeros((B, k + 1), dtype=torch.int64, device=dev)
        self.u_draft = torch.zeros((k, B), dtype=torch.float32, device=dev)
        self.u_acc = torch.zeros((B, k), dtype=torch.float32, device=dev)
        self.u_fin = torch.zeros(B, dtype=torch.float32, device=dev)
        self.conf = torch.ones(B, dtype=torch.float32, device=dev)
        self.k_used = torch.zeros(1, dtype=torch.int64, device=dev)
        # draft-step outputs: one slot per draft position, the last for the first token
        self.step_out = [(torch.zeros(B, dtype=torch.int64, device=dev),
                          torch.zeros(B, dtype=torch.float32, device=dev),
                          torch.zeros(1, dtype=torch.int32, device=dev))
                         for _ in range(k + 1)]
        self.n_acc = self.y = None
        self.last_target_logits = None
        self.last_k = 0
        L = _lib.lib()
        dcode = _lib.dtype_code(self.dlog)
        # one workspace per draft position: each keeps its rows' statistics for the
        # verify (`Verifier.drafted`), which then streams the target rows alone
        self.draft_ws = [_lib.workspace(L.sdx_draft_step_workspace(B, V, dcode), dev)
                         for _ in range(k)]
        self._verifiers = {}
        self._graphs = {}
        self.controller = controller
        self.rounds = 0
        self._out_ok = bool(getattr(draft, "writes_out", False))
        # observed cost ratio for the controller (0: keep c), from event timings
        self.c_obs = torch.zeros(1, dtype=torch.float32, device=dev)
        self.observe_cost = bool(observe_cost) and controller is not None
        self._timing = None
        self._t_draft = self._t_target = 0.0
        self._n_draft = self._n_target = 0

    def _verifier(self, k):
        v = self._verifiers.get(k)
        if v is None:
            v = Verifier(self.B, k, self.V, self.dtype, temperature=self.temperature,
                         top_p=self.top_p, top_k=self.top_k, device=self.device)
            self._verifiers[k] = v
        return v

    # ---- start: prefill and the first token (`engine.py:212-226`)
    def start(self, prompt, plen=None, u_first=None):
        """prompt [B, P] int64 on the device, right-padded; plen [B] the real prompt
        lengths (None: all P). The first token comes from the target alone at each
        row's last real position (greedy: its argmax; else a draw on u_first [B])."""
        B, P = prompt.shape
        if B != self.B:
            raise ValueError(f"prompt has {B} rows, the engine {self.B}")
        need = P + self.max_new + self.k + 1
        if need > self.capacity:
            raise ValueError(f"prompt length {P} + max_new {self.max_new} + k {self.k} + 1 "
                             f"exceeds the cache capacity {self.capacity}: pass capacity or "
                             "prompt_len to SpecEngine")
        if plen is None:
            plen = torch.full((B,), P, dtype=torch.int64)
        plen = torch.as_tensor(plen, dtype=torch.int64)
        if plen.numel() != B or int(plen.min()) < 1 or int(plen.max()) > P:
            raise ValueError("plen must hold B lengths in [1, P]")
        self.err.zero_()
        for c in (self.tcache, self.dcache):                    # a fresh sequence per row
            if hasattr(c, "set_lengths"):
                c.set_lengths(torch.zeros(B, dtype=torch.int64))
            else:
                c.lengths.zero_()
        tlog = self.target.prefill(prompt, self.tcache, plen)
        self.draft.prefill(prompt, self.dcache, plen)
        x, _, _ = draft_step(tlog.contiguous(), u_first, self.T, self.tp, self.tk,
                             out=self.step_out[self.k], workspace=self.draft_ws[0])
        # a first token that could not be drawn (nonfinite prefill logits) raises
        # the round-commit error word, read at the next sync
        self.err[0:1].bitwise_or_((x < 0).any().view(1).to(torch.int32) * 2)
        self.pending.copy_(x)
        self.out.zero_()
        self.out[:, 0].copy_(x)
        self.out_len.fill_(1)
        if self.n_eos:                                          # engine.py:225-226
            self.done.copy_(torch.isin(x, self.eos))
        else:
            self.done.zero_()
        if self.max_new <= 1:
            self.done.fill_(1)

    # ---- one round, device work only (save the early-exit reads)
    def round(self, k=None):
        """One round drafting at most k tokens (default: self.k). Returns
        (n_acc [B], y [B]) device tensors, valid until the next round."""
        B = self.B
        kr = self.k if k is None else int(k)
        if not 1 <= kr <= self.k:
            raise ValueError(f"round k {kr} outside [1, {self.k}]")
        early = self.tau is not None
        capturing = torch.cuda.is_current_stream_capturing()
        if early and capturing:
            raise RuntimeError("the confidence early exit reads the device: not capturable")
        if early:
            self.conf.fill_(1.0)
        timing = None
        if self.observe_cost and not capturing:
            timing = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
            timing[0].record()
        feed = self.pending.view(B, 1)
        k_eff = kr
        for i in range(kr):                                     # engine.py:246-258
            if self._out_ok:   # the draft writes its logits into dlog[:, i] itself
                self.draft.forward(feed, self.dcache, out=self.dlog[:, i:i + 1])
            else:
                self.dlog[:, i].copy_(self.draft.forward(feed, self.dcache)[:, -1])
            self.dcache.commit(1)
            x, _, stop = draft_step(self.dlog[:, i], self.u_draft[i], self.T, self.tp, self.tk,
                                    conf=self.conf if early else None,
                                    tau=self.tau if early else None, step=i + 1,
                                    min_k=self.min_k, out=self.step_out[i],
                                    workspace=self.draft_ws[i])
            self.xs[:, i].copy_(x)
            feed = x.view(B, 1)
            if early and i + 1 < kr and bool(stop.item()):     # controller.py:184-187
                k_eff = i + 1
                break
        self.draft.forward(feed, self.dcache)                   # commit-only forward
        self.dcache.commit(1)
        self.vin[:, 0].copy_(self.pending)                      # engine.py:266-270
        self.vin[:, 1:k_eff + 1].copy_(self.xs[:, :k_eff])
        vin = self.vin if k_eff == self.k else self.vin[:, :k_eff + 1].contiguous()
        if timing is not None:
            timing[1].record()
            timing[2].record()
        tlog = self.target.forward(vin, self.tcache)
        if timing is not None:
            timing[3].record()
            self._timing = (timing, k_eff + 1)
        self.tcache.commit(k_eff + 1)
        self.last_target_logits = tlog
        if k_eff == self.k:
            xs, dlog, ua = self.xs, self.dlog, self.u_acc
        else:
            xs = self.xs[:, :k_eff].contiguous()
            dlog = self.dlog[:, :k_eff].contiguous()
            ua = self.u_acc[:, :k_eff].contiguous()
        torch.sub(1, self.done, out=self.active)                # alive = ~done
        # engine.py:281-303, with q's statistics from this round's draft steps
        n_acc, y, flags = self._verifier(k_eff).drafted(tlog.contiguous(), dlog, xs, ua,
                                                        self.u_fin, self.draft_ws[:k_eff],
                                                        self.active)
        rc = _lib.lib().sdx_round_commit(                       # engine.py:305-340
            B, k_eff, None, _lib.ptr(n_acc), _lib.ptr(y), _lib.ptr(xs), _lib.ptr(self.done),
            _lib.ptr(self.out), _lib.ptr(self.out_len), self.max_new, _lib.ptr(self.eos),
            self.n_eos, _lib.ptr(self.tcache.lengths), _lib.ptr(self.dcache.lengths),
            _lib.ptr(self.pending), _lib.ptr(flags), _lib.ptr(self.err),
            _lib.stream_of(self.pending))
        _lib.check(rc, "SpecEngine.round")
        for c in (self.tcache, self.dcache):                    # lengths moved on the device
            moved = getattr(c, "device_rolled_back", None)
            if moved is not None:
                moved()
        if self.controller is not None:                         # controller.py:143-154
            self.k_used.fill_(k_eff)
            self.controller.update(n_acc, self.k_used,
                                   c_obs=self.c_obs if self.observe_cost else None)
        self.n_acc, self.y, self.last_k = n_acc, y, k_eff
        self.rounds += 1
        return n_acc, y

    def capture(self, k=None):
        """One round at k drafts in a HIP graph, kept for `replay(k)`. Run an
        eager round at this k first (library handles, workspaces and the
        prepared verifier are created outside the capture)."""
        if self.tau is not None:
            raise RuntimeError("the confidence early exit reads the device: not capturable")
        kr = self.k if k is None else int(k)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.round(kr)
        self.rounds -= 1
        self._graphs[kr] = (g, self.n_acc, self.y, self.last_target_logits)
        return g

    def replay(self, k=None):
        """Replay the captured round at k (after filling the uniform buffers)."""
        kr = self.k if k is None else int(k)
        g, n_acc, y, tlog = self._graphs[kr]
        g.replay()
        self.n_acc, self.y, self.last_target_logits, self.last_k = n_acc, y, tlog, kr
        self.rounds += 1
        return n_acc, y

    # ---- the generation loop (`engine.py:197-342`)
    def generate(self, prompt, plen=None, seed=0, graphs=False, max_rounds=None, on_round=None):
        """Decode right-padded prompt [B, P] with real lengths plen [B] (None: all
        P) to the end (every row at EOS or max_new tokens).
        Uniforms come from one device generator seeded with `seed`, drawn in a
        fixed order per round (u_draft, u_acc, u_fin) at the full k. With
        graphs=True every k is run eagerly once, then captured and replayed.
        on_round(engine) is called after each round (for checks). Returns the
        emitted tokens of every row."""
        g = torch.Generator(device=self.device).manual_seed(int(seed))
        u_first = torch.rand(self.B, generator=g, device=self.device)
        self.start(prompt, plen, u_first)
        n = 0
        while not self.all_done():
            if max_rounds is not None and n >= max_rounds:
                break
            k = self.k if self.controller is None else max(1, min(self.k, int(self.controller.k[0])))
            torch.rand(self.u_draft.shape, generator=g, device=self.device, out=self.u_draft)
            torch.rand(self.u_acc.shape, generator=g, device=self.device, out=self.u_acc)
            torch.rand(self.u_fin.shape, generator=g, device=self.device, out=self.u_fin)
            if graphs and self.tau is None:
                if k in self._graphs:
                    self.replay(k)
                else:
                    self.round(k)
                    self.capture(k)
            else:
                self.round(k)
            if on_round is not None:
                on_round(self)
            n += 1
        return self.outputs()

    # ---- host reads
    def sync(self):
        """The round's one host read: whether every row is done, the error words,
        and the host lengths of caches that keep them. Raises RuntimeError when a
        round commit or cache kernel set its error word."""
        mirrors = [c for c in (self.tcache, self.dcache) if hasattr(c, "set_host_lengths")]
        parts = [self.done.all().view(1).to(torch.int64), self.err.to(torch.int64)]
        parts += [c.lengths.view(-1) for c in mirrors]
        v = torch.cat(parts).cpu()
        off = 4
        for c in mirrors:
            c.set_host_lengths(v[off:off + self.B])
            off += self.B
        if self._timing is not None:
            (ev, nt), self._timing = self._timing, None
            self._t_draft += ev[0].elapsed_time(ev[1])
            self._n_draft += nt                                 # k_eff + 1 draft forwards
            self._t_target += ev[2].elapsed_time(ev[3])
            self._n_target += 1
            if self._t_target > 0.0:
                ratio = (self._t_draft / self._n_draft) / (self._t_target / self._n_target)
                self.c_obs.fill_(float(ratio))
        e0, e1, e2 = (int(x) for x in v[1:4])
        if e0 or e1 or e2:
            if e0 & 1:  # a WORKSPACE flag marks the verifier's workspace: prepare it again
                for ver in self._verifiers.values():
                    if not ver.greedy:
                        ver.reset_workspace()
            what = []
            if e0 & 1:
                what.append("a live row was flagged NONFINITE, UNSUPPORTED, BAD_ROW or WORKSPACE")
            if e0 & 2:
                what.append("a live row got no token (y < 0)")
            if e1:
                what.append("the target cache overflowed or rolled back below zero")
            if e2:
                what.append("the draft cache overflowed or rolled back below zero")
            self.err.zero_()
            raise RuntimeError("SpecEngine: " + "; ".join(what))
        return bool(v[0])

    def all_done(self):
        return self.sync()

    def outputs(self):
        """The emitted tokens of every row (one device read)."""
        out, n = self.out.cpu(), self.out_len.cpu()
        return [out[b, :min(int(n[b]), self.max_new)].tolist() for b in range(self.B)]


def autoregressive(model, prompt, max_new, eos_ids=(), capacity=None, seed=0, plen=None):
    """Greedy decoding with the target alone through the same cache, attention and
    argmax kernels (`engine.py:347-381`, generate_autoregressive): the G2
    baseline. prompt [B, P] right-padded, plen [B] its real lengths (None: P).
    Returns the emitted tokens of every row."""
    B, P = prompt.shape
    if plen is None:
        plen = torch.full((B,), P, dtype=torch.int64)
    cache = model.new_cache(B, capacity or (P + max_new + 2), seed=seed)
    logits = model.prefill(prompt, cache, torch.as_tensor(plen, dtype=torch.int64))
    eos = set(int(e) for e in eos_ids)
    out = [[] for _ in range(B)]
    done = [False] * B
    for _ in range(max_new):
        x, _, _ = draft_step(logits.contiguous(), None, 0.0)
        xl = x.tolist()
        for b in range(B):
            if done[b]:
                continue
            out[b].append(xl[b])
            if xl[b] in eos or len(out[b]) >= max_new:
                done[b] = True
        if all(done):
            break
        logits = model.forward(x.view(B, 1), cache)[:, -1]
        cache.commit(1)
    return out

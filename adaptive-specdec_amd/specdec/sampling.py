"""Sampling transforms and exact rejection sampling on MI355X.

Drop-in for the reference's `specdec/sampling.py` (`to_probs`,
`sample_from_probs`, `residual_probs`, `gather_prob`, `__all__` at :31) plus
`rejection_sample`, the accept block of `specdec/engine.py:285-303` as one
call. Every function runs hand-written HIP kernels through
libspecdec_amd.so; tensors must be on the ROCm device.

Semantics follow the reference exactly where torch is deterministic and fix a
rule where it is not:
* transform order `sampling.py:42-67`: fp32 cast, greedy one-hot (first index
  among maxima) for T <= 0, softmax(l / T), top-k zeroing without
  renormalisation, top-p keep test `cum - p < top_p` on the top-k-zeroed
  probabilities with the first token always kept, renormalise;
* ties inside the top-p boundary group keep the lowest token ids (the
  reference's CPU sort is unstable, so it leaves this unspecified);
* the softmax numerator is exp_det(s - m) with s = fl32(l / T): a float64
  Cody-Waite reduction, then the degree-9 Taylor polynomial of exp in fp32
  Horner form (plain multiply then add), scaled by a power of two; the
  normaliser and all masses are exact 2^-62 fixed-point sums, so decisions do
  not depend on summation order;
* sampling is an inverse-CDF draw on a uniform instead of torch.multinomial's
  exponential race: the same distribution, reproducible ids.
"""
import torch

from . import _lib

__all__ = ["to_probs", "sample_from_probs", "residual_probs", "gather_prob", "rejection_sample",
           "rejection_sample_ragged", "Verifier", "draft_step"]

# per-row flags of the verify calls (the SDX_FLAG_* bits of the C ABI)
FLAG_ACCEPT_NEAR_TIE = 1   # an evaluated accept test had |u - min(p/q, 1)| < 1e-5
FLAG_NONFINITE = 2         # a logit row held +inf or NaN
FLAG_UNSUPPORTED = 4       # a row's mass spans more distinct values than the kernels represent
FLAG_BAD_ROW = 8           # per-row k: inconsistent offsets
FLAG_WORKSPACE = 16        # workspace not prepared, or a draw's bounded wait gave up
FLAG_TIE_ORDER = 32        # a test or the draw touched a partially kept top-p tie group


def _switch_args(temperature, top_p, top_k):
    T = 0.0 if temperature is None or temperature <= 0.0 else float(temperature)
    tp = float(top_p) if (top_p is not None and 0.0 < top_p < 1.0) else 1.0
    tk = int(top_k) if top_k else 0
    return T, tp, tk


def _kernel_rows(x):
    """[rows, V] in a layout the row kernels accept: fp32/bf16/fp16, rows
    starting 16-byte aligned with a stride that is a multiple of 8 (16-bit) or
    4 (fp32) elements. Returns (tensor, ld)."""
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        x = x.float()                      # sampling.py:42 upcasts anything else
    x = _lib.widen_f16(x)
    V = x.shape[-1]
    mult = 4 if x.dtype == torch.float32 else 8
    if x.is_contiguous() and V % mult == 0 and x.data_ptr() % 16 == 0:
        return x, V
    if (x.dim() == 2 and x.stride(1) == 1 and x.stride(0) >= V and x.stride(0) % mult == 0
            and V % mult == 0 and x.data_ptr() % 16 == 0):
        return x, x.stride(0)              # rows of a wider buffer, read in place
    ld = (V + mult - 1) // mult * mult
    buf = torch.empty((x.shape[0], ld), dtype=x.dtype, device=x.device)
    buf[:, :V].copy_(x)
    return buf, ld


def to_probs(logits, temperature=1.0, top_p=1.0, top_k=0):
    """Logits [..., V] -> fp32 probabilities [..., V] (`sampling.py:34-67`)."""
    _lib.require_gpu(logits)
    L = _lib.lib()
    shape = logits.shape
    V = shape[-1]
    x, ld = _kernel_rows(logits.reshape(-1, V))
    rows = x.shape[0]
    out = torch.empty((rows, V), dtype=torch.float32, device=x.device)
    if rows == 0:
        return out.reshape(shape)
    T, tp, tk = _switch_args(temperature, top_p, top_k)
    dt = _lib.dtype_code(x)
    ws = _lib.cached_workspace(L.sdx_to_probs_workspace(rows, V, dt), x.device, "to_probs")
    rc = L.sdx_to_probs(_lib.ptr(x), dt, rows, V, ld, T, tp, tk, _lib.ptr(out), V,
                        _lib.ptr(ws), ws.numel(), _lib.stream_of(x))
    _lib.check(rc, "to_probs")
    return out.reshape(shape)


def sample_from_probs(probs, generator=None, u=None):
    """One draw per row of probs [..., V] -> ids [...] (`sampling.py:70-74`).

    The draw is inverse-CDF on a uniform per row; `u` (fp32 [...], in [0, 1))
    may be given, otherwise it is drawn with `torch.rand(..., generator=generator)`.
    """
    _lib.require_gpu(probs)
    L = _lib.lib()
    V = probs.shape[-1]
    p, ld = _kernel_rows(probs.reshape(-1, V).float())
    rows = p.shape[0]
    if u is None:
        u = torch.rand(rows, device=p.device, generator=generator)
    u = u.reshape(-1).to(torch.float32).contiguous()
    ids = torch.empty(rows, dtype=torch.int64, device=p.device)
    if rows:
        ws = _lib.cached_workspace(L.sdx_sample_probs_workspace(rows, V), p.device, "sample")
        rc = L.sdx_sample_probs(_lib.ptr(p), rows, V, ld, _lib.ptr(u), _lib.ptr(ids),
                                _lib.ptr(ws), ws.numel(), _lib.stream_of(p))
        _lib.check(rc, "sample_from_probs")
    return ids.reshape(probs.shape[:-1])


def residual_probs(p, q):
    """norm((p - q)_+), p where that mass is <= 1e-9 (`sampling.py:77-90`)."""
    _lib.require_gpu(p, q)
    L = _lib.lib()
    V = p.shape[-1]
    pp, ld = _kernel_rows(p.reshape(-1, V).float())
    qq, ldq = _kernel_rows(q.reshape(-1, V).float())
    if ldq != ld:
        raise ValueError("p and q must have the same shape")
    rows = pp.shape[0]
    out = torch.empty((rows, V), dtype=torch.float32, device=pp.device)
    if rows:
        ws = _lib.cached_workspace(L.sdx_residual_probs_workspace(rows, V), pp.device, "residual")
        rc = L.sdx_residual_probs(_lib.ptr(pp), _lib.ptr(qq), rows, V, ld, _lib.ptr(out), V,
                                  _lib.ptr(ws), ws.numel(), _lib.stream_of(pp))
        _lib.check(rc, "residual_probs")
    return out.reshape(p.shape)


def gather_prob(probs, ids):
    """probs [..., V], ids [...] -> probs at ids, shape [...] (`sampling.py:93-95`)."""
    _lib.require_gpu(probs, ids)
    L = _lib.lib()
    V = probs.shape[-1]
    p = probs.reshape(-1, V).float().contiguous()
    i = ids.reshape(-1).to(torch.int64).contiguous()
    if i.numel() != p.shape[0]:
        raise ValueError("ids must have the leading shape of probs")
    out = torch.empty(p.shape[0], dtype=torch.float32, device=p.device)
    if p.shape[0]:
        rc = L.sdx_gather_prob(_lib.ptr(p), p.shape[0], V, V, _lib.ptr(i), _lib.ptr(out),
                               _lib.stream_of(p))
        _lib.check(rc, "gather_prob")
    return out.reshape(ids.shape)


def rejection_sample(target_logits, draft_logits, draft_ids, u_accept, u_final, *,
                     temperature=1.0, top_p=1.0, top_k=0, active=None, out=None):
    """The verify step of `engine.py:281-303` in one device call.

    target_logits [B, k+1, V] and draft_logits [B, k, V] (fp32/bf16/fp16; the
    same transform is applied to both, `sampling.py:5-19`), draft_ids [B, k],
    u_accept [B, k] (the per-position uniforms of `engine.py:291`), u_final [B]
    (the residual/bonus draw), active [B] bool (the engine's ~done; None = all).
    Returns (n_acc [B] int64, y [B] int64, flags [B] uint8): row b emits
    draft_ids[b, :n_acc[b]] then y[b] and drops k - n_acc[b] cached positions.
    flags bit 0 marks rows whose accept decision was within 1e-5 of flipping;
    bit 1 rows with +inf/NaN logits and bit 2 rows outside the kernels'
    histogram windows (both: results of that row unspecified).
    With temperature <= 0 the draft logits are not read (may be None).
    """
    T, tp, tk = _switch_args(temperature, top_p, top_k)
    greedy = T == 0.0
    _lib.require_gpu(target_logits, draft_ids, u_accept, u_final,
                     None if greedy else draft_logits, active)
    L = _lib.lib()
    B, k1, V = target_logits.shape
    k = k1 - 1
    if k < 1:
        raise ValueError("need at least one draft position (target is [B, k+1, V])")
    dev = target_logits.device
    tl = target_logits
    if tl.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        tl = tl.float()
    dl = None if greedy else draft_logits.to(tl.dtype)
    if not greedy and tuple(dl.shape) != (B, k, V):
        raise ValueError(f"draft_logits must be [{B}, {k}, {V}], got {tuple(dl.shape)}")
    if tl.dtype != torch.float32 and (V % 8 != 0 or _lib.widen_f16(tl) is not tl):
        # 16-bit rows must be 16-byte aligned and fp16 rows at most F16_MAX_VOCAB
        # long; the fp32 path takes any vocab it supports
        tl = tl.float()
        dl = None if dl is None else dl.float()
    tl = tl.contiguous()
    dl = None if dl is None else dl.contiguous()
    ids = draft_ids.to(torch.int64).contiguous()
    ua = u_accept.to(torch.float32).contiguous()
    uf = u_final.to(torch.float32).contiguous()
    act = None if active is None else active.to(torch.uint8).contiguous()
    if out is None:
        n_acc = torch.empty(B, dtype=torch.int64, device=dev)
        y = torch.empty(B, dtype=torch.int64, device=dev)
        flags = torch.empty(B, dtype=torch.uint8, device=dev)
    else:
        n_acc, y, flags = out
    if B == 0:
        return n_acc, y, flags
    dt = _lib.dtype_code(tl)
    st = _lib.stream_of(tl)
    if greedy:
        ws = _lib.cached_workspace(L.sdx_verify_greedy_workspace(B, k), dev, "greedy")
        rc = L.sdx_verify_greedy(_lib.ptr(tl), dt, B, k, V, _lib.ptr(ids), _lib.ptr(ua),
                                 _lib.ptr(act), _lib.ptr(n_acc), _lib.ptr(y), _lib.ptr(flags),
                                 _lib.ptr(ws), ws.numel(), st)
    else:
        ws = _lib.cached_workspace(L.sdx_verify_workspace(B, k, V, dt), dev, "verify")
        rc = L.sdx_verify(_lib.ptr(tl), _lib.ptr(dl), dt, B, k, V, _lib.ptr(ids), _lib.ptr(ua),
                          _lib.ptr(uf), _lib.ptr(act), T, tp, tk, _lib.ptr(n_acc), _lib.ptr(y),
                          _lib.ptr(flags), _lib.ptr(ws), ws.numel(), st)
    _lib.check(rc, "rejection_sample")
    return n_acc, y, flags


def rejection_sample_ragged(target_logits, draft_logits, draft_ids, u_accept, u_final, cu_k, *,
                            k_max=None, temperature=1.0, top_p=1.0, top_k=0, active=None,
                            workspace=None, out=None):
    """`rejection_sample` with a different k per batch row (adaptive k per row).

    Row b drafts k_b = cu_k[b+1] - cu_k[b] tokens (cu_k int64 [B+1], cu_k[0] = 0).
    Rows are packed: target_logits [sum(k_b+1), V] with row b's positions at
    cu_k[b] + b, draft_logits [sum k_b, V], draft_ids and u_accept [sum k_b] with
    row b's at cu_k[b]; u_final [B]. k_max bounds every k_b (None: read from cu_k,
    one host sync). Returns (n_acc, y, flags) as `rejection_sample`: row b emits
    draft_ids[cu_k[b] : cu_k[b] + n_acc[b]] then y[b] and drops k_b - n_acc[b]
    cached positions. Offsets that are inconsistent set FLAG_BAD_ROW on every row.
    """
    T, tp, tk = _switch_args(temperature, top_p, top_k)
    greedy = T == 0.0
    _lib.require_gpu(target_logits, draft_ids, u_accept, u_final, cu_k,
                     None if greedy else draft_logits, active)
    L = _lib.lib()
    NT, V = target_logits.shape
    B = cu_k.numel() - 1
    if NT < B:
        raise ValueError(f"target_logits has {NT} rows, fewer than the {B} batch rows")
    cu = cu_k.to(torch.int64).contiguous()
    if k_max is None:
        k_max = int((cu[1:] - cu[:-1]).max().item()) if B > 0 else 1
    k_max = max(int(k_max), 1)
    dev = target_logits.device
    tl = target_logits
    if tl.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        tl = tl.float()
    dl = None if greedy else draft_logits.to(tl.dtype)
    if not greedy and tuple(dl.shape) != (NT - B, V):
        raise ValueError(f"draft_logits must be [{NT - B}, {V}], got {tuple(dl.shape)}")
    if tl.dtype != torch.float32 and (V % 8 != 0 or _lib.widen_f16(tl) is not tl):
        tl = tl.float()
        dl = None if dl is None else dl.float()
    tl = tl.contiguous()
    if greedy:
        dl = tl  # not read; the C ABI wants a pointer of the right type
    dl = dl.contiguous()
    ids = draft_ids.to(torch.int64).contiguous()
    ua = u_accept.to(torch.float32).contiguous()
    uf = u_final.to(torch.float32).contiguous()
    if ids.numel() != NT - B or ua.numel() != NT - B or uf.numel() != B:
        raise ValueError("draft_ids / u_accept must hold sum(k_b) entries and u_final B")
    act = None if active is None else active.to(torch.uint8).contiguous()
    if out is None:
        n_acc = torch.empty(B, dtype=torch.int64, device=dev)
        y = torch.empty(B, dtype=torch.int64, device=dev)
        flags = torch.empty(B, dtype=torch.uint8, device=dev)
    else:
        n_acc, y, flags = out
    if B == 0:
        return n_acc, y, flags
    dt = _lib.dtype_code(tl)
    need = L.sdx_verify_ragged_workspace(B, NT, V, dt)
    if workspace is None or workspace.numel() < need:
        workspace = _lib.cached_workspace(need, dev, "verify")
    rc = L.sdx_verify_ragged(_lib.ptr(tl), _lib.ptr(dl), dt, B, k_max, NT, V, _lib.ptr(cu),
                             _lib.ptr(ids), _lib.ptr(ua), _lib.ptr(uf), _lib.ptr(act), T, tp, tk,
                             _lib.ptr(n_acc), _lib.ptr(y), _lib.ptr(flags), _lib.ptr(workspace),
                             workspace.numel(), _lib.stream_of(tl))
    _lib.check(rc, "rejection_sample_ragged")
    return n_acc, y, flags


class Verifier:
    """`rejection_sample` prepared for fixed shapes: workspace and outputs are
    allocated once, each call is one C-ABI call (capturable in a HIP graph).

    v = Verifier(B, k, V, torch.bfloat16, temperature=0.8, top_p=0.95)
    n_acc, y, flags = v(target, draft, draft_ids, u_accept, u_final)
    """

    def __init__(self, batch, k, vocab, dtype, temperature=1.0, top_p=1.0, top_k=0,
                 device="cuda"):
        self.B, self.k, self.V = int(batch), int(k), int(vocab)
        self.T, self.tp, self.tk = _switch_args(temperature, top_p, top_k)
        self.greedy = self.T == 0.0
        self.dt = _lib.dtype_code(torch.empty(0, dtype=dtype))
        if self.dt != _lib.F32 and self.V % 8 != 0:
            raise ValueError("16-bit logits need vocab % 8 == 0 for the prepared path")
        self.dtype = dtype
        L = _lib.lib()
        self.L = L
        dev = torch.device(device)
        # fp16 rows longer than the fp16 kernels take: each call copies them into
        # fp32 buffers allocated here (exact) and runs the fp32 kernels
        self._t32 = self._d32 = None
        if self.dt == _lib.F16 and self.V > _lib.F16_MAX_VOCAB:
            self.dt = _lib.F32
            self._t32 = torch.empty((self.B, self.k + 1, self.V), dtype=torch.float32, device=dev)
            if not self.greedy:
                self._d32 = torch.empty((self.B, self.k, self.V), dtype=torch.float32, device=dev)
        nbytes = (L.sdx_verify_greedy_workspace(self.B, self.k) if self.greedy
                  else L.sdx_verify_workspace(self.B, self.k, self.V, self.dt))
        self.ws = _lib.workspace(nbytes, dev)
        self.n_acc = torch.empty(self.B, dtype=torch.int64, device=dev)
        self.y = torch.empty(self.B, dtype=torch.int64, device=dev)
        self.flags = torch.empty(self.B, dtype=torch.uint8, device=dev)

    def _check(self, target, draft, ids, ua, uf):
        if target.dtype != self.dtype or tuple(target.shape) != (self.B, self.k + 1, self.V):
            raise ValueError("target does not match the prepared shape/dtype")
        if not self.greedy and (draft.dtype != self.dtype or
                                tuple(draft.shape) != (self.B, self.k, self.V)):
            raise ValueError("draft does not match the prepared shape/dtype")
        for t, dt in ((ids, torch.int64), (ua, torch.float32), (uf, torch.float32)):
            if t.dtype != dt or not t.is_contiguous():
                raise ValueError("draft_ids int64, u_accept/u_final fp32, all contiguous")
        for t in (target, draft):
            if t is not None and not t.is_contiguous():
                raise ValueError("logits must be contiguous")

    def _rows(self, target, draft):
        """The logits the kernels read: the caller's, or their fp32 copies."""
        if self._t32 is None:
            return target, draft
        self._t32.copy_(target)
        if self._d32 is not None:
            self._d32.copy_(draft)
        return self._t32, self._d32

    def __call__(self, target, draft, draft_ids, u_accept, u_final, active=None):
        self._check(target, draft, draft_ids, u_accept, u_final)
        act = None if active is None else active.to(torch.uint8)
        st = _lib.stream_of(target)
        target, draft = self._rows(target, draft)
        if self.greedy:
            rc = self.L.sdx_verify_greedy(_lib.ptr(target), self.dt, self.B, self.k, self.V,
                                          _lib.ptr(draft_ids), _lib.ptr(u_accept), _lib.ptr(act),
                                          _lib.ptr(self.n_acc), _lib.ptr(self.y),
                                          _lib.ptr(self.flags), _lib.ptr(self.ws),
                                          self.ws.numel(), st)
        else:
            rc = self.L.sdx_verify(_lib.ptr(target), _lib.ptr(draft), self.dt, self.B, self.k,
                                   self.V, _lib.ptr(draft_ids), _lib.ptr(u_accept),
                                   _lib.ptr(u_final), _lib.ptr(act), self.T, self.tp, self.tk,
                                   _lib.ptr(self.n_acc), _lib.ptr(self.y), _lib.ptr(self.flags),
                                   _lib.ptr(self.ws), self.ws.numel(), st)
        _lib.check(rc, "Verifier")
        return self.n_acc, self.y, self.flags

    def drafted(self, target, draft, draft_ids, u_accept, u_final, draft_workspaces,
                active=None):
        """The same call as `__call__` for a round whose k draft rows went through
        `draft_step`: draft_workspaces[i] is the workspace of the draft step that
        drew draft_ids[:, i] from draft[:, i]. The draft rows' statistics are taken
        from there instead of streaming draft again (bf16 at T > 0; other cases
        verify as `__call__`). Same results as `__call__`."""
        import ctypes
        self._check(target, draft, draft_ids, u_accept, u_final)
        if len(draft_workspaces) != self.k:
            raise ValueError(f"need {self.k} draft workspaces, got {len(draft_workspaces)}")
        if self.greedy:
            return self(target, draft, draft_ids, u_accept, u_final, active)
        act = None if active is None else active.to(torch.uint8)
        target, draft = self._rows(target, draft)
        arr = (ctypes.c_void_p * self.k)(*[w.data_ptr() for w in draft_workspaces])
        rc = self.L.sdx_verify_drafted(_lib.ptr(target), _lib.ptr(draft), self.dt, self.B, self.k,
                                       self.V, _lib.ptr(draft_ids), _lib.ptr(u_accept),
                                       _lib.ptr(u_final), _lib.ptr(act), self.T, self.tp, self.tk,
                                       ctypes.cast(arr, ctypes.c_void_p), _lib.ptr(self.n_acc),
                                       _lib.ptr(self.y), _lib.ptr(self.flags), _lib.ptr(self.ws),
                                       self.ws.numel(), _lib.stream_of(target))
        _lib.check(rc, "Verifier.drafted")
        return self.n_acc, self.y, self.flags

    def reset_workspace(self):
        """Prepare the workspace again: after rows came back FLAG_WORKSPACE (a
        draw's bounded wait gave up and marked the workspace header), every later
        call flags its rows until this runs."""
        _lib.prepare(self.ws)

    def stats(self, target, draft, draft_ids=None):
        """Phase 1 only (fused to_probs statistics of all rows), for timing.
        Without draft_ids: the row statistics alone (no gathered probabilities)."""
        if self.greedy:
            raise ValueError("greedy verify has no statistics phase")
        ids = _lib.ptr(draft_ids) if draft_ids is not None else None
        target, draft = self._rows(target, draft)
        rc = self.L.sdx_verify_stats(_lib.ptr(target), _lib.ptr(draft), self.dt, self.B, self.k,
                                     self.V, ids, self.T, self.tp, self.tk,
                                     _lib.ptr(self.ws), self.ws.numel(), _lib.stream_of(target))
        _lib.check(rc, "Verifier.stats")


def draft_step(logits, u, temperature=1.0, top_p=1.0, top_k=0, conf=None, tau=None, step=1,
               min_k=1, out=None, workspace=None):
    """One draft step of `engine.py:246-258` in one device call.

    logits [B, V] (the draft's last position), u [B] fp32 uniforms of the draw.
    q = to_probs(logits) (`sampling.py:34-67`); x = the inverse-CDF draw from q
    on u (the rule of `sample_from_probs`; T <= 0: the first argmax); qx = q(x).
    conf [B] fp32 (optional) is multiplied by qx in place (`engine.py:256`); with
    tau given, stop [1] int32 is set on the device to the early-exit test of
    `controller.py:184-187`: step >= min_k and mean(conf) < tau. Returns
    (x [B] int64, qx [B] fp32, stop [1] int32 or None); nothing waits for the host.
    """
    T, tp, tk = _switch_args(temperature, top_p, top_k)
    _lib.require_gpu(logits, None if T == 0.0 else u, conf)
    L = _lib.lib()
    B, V = logits.shape
    x_in, ld = _kernel_rows(logits)
    dt = _lib.dtype_code(x_in)
    dev = logits.device
    if out is None:
        x = torch.empty(B, dtype=torch.int64, device=dev)
        qx = torch.empty(B, dtype=torch.float32, device=dev)
        stop = torch.zeros(1, dtype=torch.int32, device=dev) if tau is not None else None
    else:
        x, qx, stop = out
    if B == 0:
        return x, qx, stop
    uu = None if T == 0.0 else u.to(torch.float32).contiguous()
    if conf is not None and (conf.dtype != torch.float32 or not conf.is_contiguous()):
        raise ValueError("conf must be a contiguous fp32 tensor (updated in place)")
    need = L.sdx_draft_step_workspace(B, V, dt)
    if workspace is None or workspace.numel() < need:
        workspace = _lib.cached_workspace(need, dev, "draft")
    rc = L.sdx_draft_step(_lib.ptr(x_in), dt, B, V, ld, T, tp, tk, _lib.ptr(uu), _lib.ptr(x),
                          _lib.ptr(qx), _lib.ptr(conf), float(tau if tau is not None else 0.0),
                          int(step), int(min_k), _lib.ptr(stop), _lib.ptr(workspace),
                          workspace.numel(), _lib.stream_of(x_in))
    _lib.check(rc, "draft_step")
    return x, qx, stop

"""Oracle restatement of `specdec/sampling.py` and the accept block of `specdec/engine.py`.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`).

Arrays are numpy; logits may be any float dtype that upcasts exactly to fp32
(bf16 and fp16 do). Every function cites the reference lines it restates.
Two rules are fixed where the reference defers to unreproducible torch
internals:

1. Top-p ties (`sampling.py:57`): torch's CPU `sort` is not stable, so which
   members of the tie group that straddles the nucleus boundary survive is
   unspecified. Here the sort is stable: among equal probabilities the lower
   token id comes first (and is kept first).
2. Sampling (`sampling.py:70-74`, `torch.multinomial`): replaced by an exact
   inverse-CDF draw on caller-supplied uniforms over fixed62 weights
   (`sample_fixed`). Same distribution, reproducible token ids.
"""
import numpy as np

from .numerics import exp_det, fixed62, fixed62_sum, rn32, rn32_u64, uniform_threshold

ACCEPT_TIE_EPS = np.float32(1e-5)
FLAG_ACCEPT_NEAR_TIE = 1
FLAG_TIE_ORDER = 32


def _enabled(temperature, top_p, top_k, V):
    """The three switches of `sampling.py:43,52,56`."""
    greedy = temperature is None or temperature <= 0.0
    use_p = top_p is not None and 0.0 < top_p < 1.0
    use_k = bool(top_k) and 0 < top_k < V
    return greedy, use_p, use_k


def _softmax_row(x, temperature):
    """`sampling.py:50`: softmax(logits / T) of one fp32 row under the exp rule."""
    s = x / np.float32(temperature)              # logits / T (fp32)
    d = s - s.max()
    e = exp_det(d)
    zf = rn32(fixed62_sum(e))
    return (e / zf).astype(np.float32)


def _transform_row(x, temperature, top_p, top_k):
    """One row of `to_probs` (`sampling.py:34-67`). x: fp32 [V]."""
    V = x.shape[0]
    greedy, use_p, use_k = _enabled(temperature, top_p, top_k, V)
    if greedy:                                   # sampling.py:43-48
        out = np.zeros(V, np.float32)
        out[int(np.argmax(x))] = 1.0             # first index among maxima
        return out
    p = _softmax_row(x, temperature)
    return filter_renorm(p, top_p if use_p else None, top_k if use_k else None)


def boundary_tie_group(x, temperature, top_p, top_k):
    """Members of the row's partially kept top-p boundary tie group, or None.

    `sampling.py:57-64` keeps a prefix of the descending sort; when the last
    kept probability v is shared by a token the nucleus drops, the tokens of
    probability v (after top-k zeroing) form a group of which only some survive,
    and torch's unstable sort decides which (here: the lowest ids). A token's
    kept probability inside such a group depends on that order. Returns a bool
    mask [V] of the group's members (kept and dropped), None when no group is
    partially kept (greedy rows, top-p off, or the cut between distinct values).
    """
    x = np.asarray(x, np.float32)
    V = x.shape[0]
    greedy, use_p, use_k = _enabled(temperature, top_p, top_k, V)
    if greedy or not use_p:
        return None
    p = _softmax_row(x, temperature)
    if use_k:
        kth = np.sort(p)[-int(top_k)]
        p = np.where(p < kth, np.float32(0.0), p)
    srt = p[np.argsort(-p, kind="stable")]
    cum = rn32_u64(np.cumsum(fixed62(srt), dtype=np.uint64))
    keep = (cum - srt) < np.float32(top_p)
    keep[0] = True
    j = int(np.count_nonzero(keep)) - 1          # keep is a prefix of the sort
    vb = srt[j]
    if j + 1 >= V or srt[j + 1] != vb or vb <= 0:
        return None
    return p == vb


def filter_renorm(p, top_p=None, top_k=None):
    """Top-k zeroing, top-p nucleus and renormalisation of `sampling.py:52-67`,
    applied to one fp32 probability row p [V]. None disables a filter."""
    V = p.shape[0]
    if top_k is not None:                        # sampling.py:52-54 (no renorm)
        kth = np.sort(p)[-int(top_k)]
        p = np.where(p < kth, np.float32(0.0), p)
    if top_p is not None:                        # sampling.py:56-64
        order = np.argsort(-p, kind="stable")    # descending; ties -> lower id first
        srt = p[order]
        cum = rn32_u64(np.cumsum(fixed62(srt), dtype=np.uint64))
        keep = (cum - srt) < np.float32(top_p)
        keep[0] = True
        mask = np.zeros(V, bool)
        mask[order] = keep
        p = np.where(mask, p, np.float32(0.0))
    total = max(rn32(fixed62_sum(p)), np.float32(1e-12))   # sampling.py:66-67
    return (p / total).astype(np.float32)


def to_probs(logits, temperature=1.0, top_p=1.0, top_k=0):
    """`to_probs` (`sampling.py:34-67`): logits [..., V] -> fp32 probs [..., V]."""
    x = np.asarray(logits, dtype=np.float32)
    flat = x.reshape(-1, x.shape[-1])
    out = np.stack([_transform_row(r, temperature, top_p, top_k) for r in flat])
    return out.reshape(x.shape)


def gather_prob(probs, ids):
    """`gather_prob` (`sampling.py:93-95`)."""
    probs = np.asarray(probs, np.float32)
    ids = np.asarray(ids, np.int64)
    return np.take_along_axis(probs, ids[..., None], axis=-1)[..., 0]


def residual_probs(p, q):
    """`residual_probs` (`sampling.py:77-90`): norm((p - q)_+), p when degenerate."""
    p = np.asarray(p, np.float32)
    q = np.asarray(q, np.float32)
    flat_p = p.reshape(-1, p.shape[-1])
    flat_q = q.reshape(-1, q.shape[-1])
    out = np.empty_like(flat_p)
    for i in range(flat_p.shape[0]):
        r = np.maximum(flat_p[i] - flat_q[i], np.float32(0.0))
        tot = rn32(fixed62_sum(r))
        if tot <= np.float32(1e-9):
            r = flat_p[i]
            tot = rn32(fixed62_sum(r))
        out[i] = r / max(tot, np.float32(1e-12))
    return out.reshape(p.shape)


def sample_fixed(weights, u):
    """Inverse-CDF draw: the first index j with prefix(w)[j] > floor(u * sum(w)).

    weights: uint64 fixed62 masses [V]; u: fp32 in [0, 1). Returns -1 for an
    all-zero row (where the reference's multinomial raises).
    """
    w = np.asarray(weights, np.uint64)
    total = int((w >> np.uint64(31)).sum(dtype=np.uint64)) << 31
    total += int((w & np.uint64((1 << 31) - 1)).sum(dtype=np.uint64))
    if total == 0:
        return -1
    t = uniform_threshold(u, total)
    cum = np.cumsum(w, dtype=np.uint64)
    return int(np.searchsorted(cum, np.uint64(t), side="right"))


def sample_from_probs(probs, u):
    """`sample_from_probs` (`sampling.py:70-74`) with explicit uniforms u [...]."""
    probs = np.asarray(probs, np.float32)
    flat = probs.reshape(-1, probs.shape[-1])
    uu = np.asarray(u, np.float32).reshape(-1)
    ids = np.array([sample_fixed(fixed62(r), uu[i]) for i, r in enumerate(flat)], np.int64)
    return ids.reshape(probs.shape[:-1])


def _residual_weights(p, q):
    """fixed62 weights of `residual_probs(p, q)` before its final division.

    Sampling the unnormalised residual by inverse CDF draws from the same
    distribution as `sample_from_probs(residual_probs(p, q))`.
    """
    r = np.maximum(p - q, np.float32(0.0))
    w = fixed62(r)
    if rn32(fixed62_sum(r)) <= np.float32(1e-9):   # sampling.py:85-88
        w = fixed62(p)
    return w


def accept_chain(px, qx, u, alive):
    """Accept loop of `engine.py:286-294` for one row.

    px, qx: fp32 [k] target/draft probs of the drafted tokens; u: fp32 [k].
    Returns (n_acc, flags). flags bit 0: some evaluated test had
    |u - min(p/q, 1)| < 1e-5 (the decision is within rounding of flipping).
    """
    n_acc, flags = 0, 0
    for i in range(len(px)):
        ratio = np.float32(px[i]) / max(np.float32(qx[i]), np.float32(1e-10))
        r1 = min(ratio, np.float32(1.0))
        evaluated = alive and n_acc == i
        ok = bool(np.float32(u[i]) < r1) and evaluated
        if evaluated and np.float32(abs(np.float32(u[i]) - r1)) < ACCEPT_TIE_EPS:
            flags |= FLAG_ACCEPT_NEAR_TIE
        n_acc += int(ok)
        alive = alive and ok
    return n_acc, flags


def rejection_sample(target_logits, draft_logits, draft_ids, u_accept, u_final,
                     temperature=1.0, top_p=1.0, top_k=0, active=None):
    """Verify step of `engine.py:281-303` on logits.

    target_logits [B, k+1, V], draft_logits [B, k, V], draft_ids [B, k] int,
    u_accept [B, k] fp32 (the engine's per-position `torch.rand(B)` draws,
    `engine.py:291`), u_final [B] fp32 (the residual/bonus draw).
    Returns (n_acc [B] int64, y [B] int64, flags [B] uint8). The tokens emitted
    for row b are draft_ids[b, :n_acc[b]] followed by y[b]; the KV drop is
    k - n_acc[b] (`engine.py:310`).

    flags: FLAG_ACCEPT_NEAR_TIE (see accept_chain); FLAG_TIE_ORDER when an
    evaluated accept test's drafted token, or y, is a member of a partially
    kept boundary tie group (`boundary_tie_group`) of a distribution it was
    tested or drawn from (p_i and q_i for test i; p_k for the bonus draw; p_n,
    and q_n unless the residual is degenerate, for the residual draw): those
    rows would read other probabilities under another order of equal values
    in torch's sort.
    """
    tl = np.asarray(target_logits, np.float32)
    dl = np.asarray(draft_logits, np.float32)
    B, k1, V = tl.shape
    k = k1 - 1
    ids = np.asarray(draft_ids, np.int64)
    ua = np.asarray(u_accept, np.float32)
    uf = np.asarray(u_final, np.float32)
    act = np.ones(B, bool) if active is None else np.asarray(active, bool)
    n_acc = np.zeros(B, np.int64)
    y = np.zeros(B, np.int64)
    flags = np.zeros(B, np.uint8)
    for b in range(B):
        ps = np.stack([_transform_row(tl[b, i], temperature, top_p, top_k) for i in range(k + 1)])
        qs = np.stack([_transform_row(dl[b, i], temperature, top_p, top_k) for i in range(k)])
        gp = [boundary_tie_group(tl[b, i], temperature, top_p, top_k) for i in range(k + 1)]
        gq = [boundary_tie_group(dl[b, i], temperature, top_p, top_k) for i in range(k)]
        px = ps[np.arange(k), ids[b]]
        qx = qs[np.arange(k), ids[b]]
        n, f = accept_chain(px, qx, ua[b], bool(act[b]))
        if act[b]:
            for i in range(min(n + 1, k)):           # the evaluated tests
                t = ids[b, i]
                if (gp[i] is not None and gp[i][t]) or (gq[i] is not None and gq[i][t]):
                    f |= FLAG_TIE_ORDER
        if n == k:                                   # bonus draw from p_{k+1}
            w = fixed62(ps[k])
            groups = [gp[k]]
        else:                                        # residual at the stop position
            w = _residual_weights(ps[n], qs[n])
            degenerate = rn32(fixed62_sum(np.maximum(ps[n] - qs[n], np.float32(0.0)))) \
                <= np.float32(1e-9)
            groups = [gp[n]] if degenerate else [gp[n], gq[n]]
        y[b] = sample_fixed(w, uf[b])
        if y[b] >= 0 and any(g is not None and g[y[b]] for g in groups):
            f |= FLAG_TIE_ORDER
        n_acc[b], flags[b] = n, f
    return n_acc, y, flags


def rejection_sample_ragged(target_logits, draft_logits, draft_ids, u_accept, u_final, cu_k,
                            temperature=1.0, top_p=1.0, top_k=0, active=None):
    """Verify with k_b = cu_k[b+1] - cu_k[b] drafts in row b: row b is the verify
    step of `engine.py:281-303` run at its own k on its packed rows (targets
    [cu_k[b] + b, + k_b + 1), drafts, ids and uniforms [cu_k[b], + k_b)); with
    k_b = 0 the row draws its bonus token from its one target row.
    Returns (n_acc [B], y [B], flags [B])."""
    tl = np.asarray(target_logits, np.float32)
    dl = None if draft_logits is None else np.asarray(draft_logits, np.float32)
    ids = np.asarray(draft_ids, np.int64)
    ua = np.asarray(u_accept, np.float32)
    uf = np.asarray(u_final, np.float32)
    cu = np.asarray(cu_k, np.int64)
    B = cu.size - 1
    act = np.ones(B, bool) if active is None else np.asarray(active, bool)
    n_acc = np.zeros(B, np.int64)
    y = np.zeros(B, np.int64)
    flags = np.zeros(B, np.uint8)
    for b in range(B):
        c0, kb = int(cu[b]), int(cu[b + 1] - cu[b])
        t = tl[c0 + b:c0 + b + kb + 1]
        if kb == 0:                                  # nothing drafted: the bonus draw
            if temperature is None or temperature <= 0:
                y[b] = argmax_first(t[0])
            else:
                y[b] = sample_fixed(fixed62(_transform_row(t[0], temperature, top_p, top_k)), uf[b])
                grp = boundary_tie_group(t[0], temperature, top_p, top_k)
                if y[b] >= 0 and grp is not None and grp[y[b]]:
                    flags[b] = FLAG_TIE_ORDER
            continue
        if temperature is None or temperature <= 0:
            n, yy, f = greedy_verify(t[None], ids[c0:c0 + kb][None], ua[c0:c0 + kb][None],
                                     act[b:b + 1])
        else:
            n, yy, f = rejection_sample(t[None], dl[c0:c0 + kb][None], ids[c0:c0 + kb][None],
                                        ua[c0:c0 + kb][None], uf[b:b + 1], temperature, top_p,
                                        top_k, act[b:b + 1])
        n_acc[b], y[b], flags[b] = n[0], yy[0], f[0]
    return n_acc, y, flags


def argmax_first(x):
    """Row-wise argmax, first index among equal maxima (torch/numpy rule)."""
    x = np.asarray(x, np.float32)
    return np.argmax(x, axis=-1).astype(np.int64)


def greedy_verify(target_logits, draft_ids, u_accept=None, active=None):
    """The T = 0 case of `rejection_sample` without draft logits.

    With one-hot p (`sampling.py:43-48`) the accept ratio p(x)/max(q(x),1e-10)
    is 0 when x is not the target argmax and >= 1 when it is, whatever q(x)
    is, so the draft logits never matter: row b accepts position i iff
    draft_ids[b, i] == argmax(target[b, i]) (and u < 1), and the emitted
    token is argmax(target[b, n_acc]) (residual of two one-hots, or the bonus
    one-hot). Returns (n_acc, y, flags).
    """
    tl = np.asarray(target_logits, np.float32)
    B, k1, V = tl.shape
    k = k1 - 1
    ids = np.asarray(draft_ids, np.int64)
    am = argmax_first(tl)                              # [B, k+1]
    ua = np.zeros((B, k), np.float32) if u_accept is None else np.asarray(u_accept, np.float32)
    act = np.ones(B, bool) if active is None else np.asarray(active, bool)
    n_acc = np.zeros(B, np.int64)
    flags = np.zeros(B, np.uint8)
    for b in range(B):
        px = (ids[b] == am[b, :k]).astype(np.float32)
        qx = np.ones(k, np.float32)
        n_acc[b], flags[b] = accept_chain(px, qx, ua[b], bool(act[b]))
    y = am[np.arange(B), n_acc]
    return n_acc, y, flags


def draft_step(logits, u, temperature=1.0, top_p=1.0, top_k=0, conf=None, tau=None, step=1,
               min_k=1):
    """One draft step, `engine.py:250-258` and `controller.py:184-187`: q =
    to_probs(logits[b]); x[b] drawn from q by `sample_fixed` on u[b] (the first
    argmax when T <= 0); qx[b] = q[b, x[b]]; conf[b] *= qx[b] in fp32; stop when
    step >= min_k and the mean of conf (a sequential fp32 sum in row order over
    B) is below tau. Returns (x, qx, conf, stop) with stop None when tau is None."""
    x_in = np.asarray(logits, np.float32)
    B = x_in.shape[0]
    greedy = temperature is None or temperature <= 0.0
    x = np.zeros(B, np.int64)
    qx = np.zeros(B, np.float32)
    for b in range(B):
        if greedy:
            x[b] = int(np.argmax(x_in[b]))
            qx[b] = np.float32(1.0)
            continue
        q = _transform_row(x_in[b], temperature, top_p, top_k)
        x[b] = sample_fixed(fixed62(q), np.float32(u[b]))
        qx[b] = q[x[b]] if x[b] >= 0 else np.float32(0.0)
    conf_out = None
    if conf is not None:
        conf_out = (np.asarray(conf, np.float32) * qx).astype(np.float32)
    stop = None
    if tau is not None:
        stop = 0
        if conf_out is not None and step >= min_k:
            s = np.float32(0.0)
            for v in conf_out:
                s = np.float32(s + v)
            stop = int(np.float32(s / np.float32(B)) < np.float32(tau))
    return x, qx, conf_out, stop

"""Seeded synthetic inputs of the verify-path workloads (no checkpoints, no data).

* verify:  B rows, k drafts, vocab V. Target logits ~ N(0, sigma^2) plus a Zipf
           boost `boost * rank^-s` on a seeded random permutation of the vocab
           per row; draft = target + N(0, draft_noise^2); draft ids drawn from
           the transformed draft distribution; fp32 uniforms for the accept
           test [B, k] and the final draw [B].
* ragged:  the verify workload with per-row k_b = best_k(alpha_b, c), alpha_b ~
           U(alpha_lo, alpha_hi), rows packed: targets [sum(k_b+1), V], drafts,
           ids and accept uniforms [sum k_b], offsets cu_k [B+1].
* greedy:  the same logits, draft ids equal to the target argmax with a given
           probability per position (else a different id).
* kv:      per-row lengths, a shuffled block table, staged K/V vectors.
* attn:    adaptive-k verify attention: per-row k from the closed-form
           controller at a per-row acceptance estimate, context lengths, a
           shuffled block table over one layer's paged K/V, queries.
"""
import torch

__all__ = ["zipf_logits", "uniforms", "verify_inputs", "ragged_verify_inputs", "greedy_inputs",
           "kv_inputs", "attn_inputs"]


def uniforms(shape, generator, device):
    """fp32 uniforms in [0, 1) on the 2^-24 grid (torch.rand's form)."""
    return torch.rand(shape, generator=generator, device=device, dtype=torch.float32)


def zipf_logits(rows, V, generator, device, sigma=3.0, boost=8.0, s=1.1, dtype=torch.bfloat16):
    x = torch.randn((rows, V), generator=generator, device=device, dtype=torch.float32) * sigma
    ranks = torch.arange(1, V + 1, device=device, dtype=torch.float32)
    bonus = boost * ranks.pow(-s)
    perm = torch.argsort(torch.rand((rows, V), generator=generator, device=device), dim=1)
    x.scatter_add_(1, perm, bonus.expand(rows, V).contiguous())
    return x.to(dtype)


def verify_inputs(B, k, V, seed, device, temperature=0.8, top_p=0.95, top_k=0, sigma=3.0,
                  draft_noise=1.0, dtype=torch.bfloat16):
    """Config of the fused-verify workload: returns a dict of device tensors."""
    from .sampling import sample_from_probs, to_probs
    g = torch.Generator(device=device).manual_seed(int(seed))
    tgt = zipf_logits(B * (k + 1), V, g, device, sigma=sigma, dtype=torch.float32)
    tgt = tgt.view(B, k + 1, V)
    noise = torch.randn((B, k, V), generator=g, device=device) * draft_noise
    drf = (tgt[:, :k] + noise).to(dtype)
    tgt = tgt.to(dtype)
    q = to_probs(drf, temperature, top_p, top_k)
    ids = sample_from_probs(q, u=uniforms((B, k), g, device))
    return {
        "target": tgt, "draft": drf, "draft_ids": ids,
        "u_accept": uniforms((B, k), g, device), "u_final": uniforms((B,), g, device),
        "temperature": temperature, "top_p": top_p, "top_k": top_k,
    }


def ragged_verify_inputs(B, V, seed, device, temperature=0.7, top_p=0.9, top_k=50, alpha_lo=0.4,
                         alpha_hi=0.9, c=0.1, k_max=8, sigma=3.0, draft_noise=1.0,
                         dtype=torch.bfloat16, k=None):
    """Adaptive-k verify: returns a dict of device tensors (packed rows) plus the
    host list of k_b. `k` (a list) overrides the controller's choice."""
    from .controller import best_k
    from .sampling import sample_from_probs, to_probs
    gc = torch.Generator(device="cpu").manual_seed(int(seed))
    if k is None:
        alphas = torch.rand(B, generator=gc) * (alpha_hi - alpha_lo) + alpha_lo
        k = [best_k(float(a), c, k_max) for a in alphas]
    k = [int(x) for x in k]
    cu = torch.zeros(B + 1, dtype=torch.int64)
    cu[1:] = torch.cumsum(torch.tensor(k, dtype=torch.int64), 0)
    nd = int(cu[-1])
    g = torch.Generator(device=device).manual_seed(int(seed))
    tgt = zipf_logits(nd + B, V, g, device, sigma=sigma, dtype=torch.float32)
    # draft row j of batch row b sits at cu[b] + j, its target position at cu[b] + b + j
    rows = torch.cat([torch.arange(int(cu[b]) + b, int(cu[b]) + b + k[b]) for b in range(B)]
                     ) if nd else torch.zeros(0, dtype=torch.int64)
    rows = rows.to(device)
    drf = (tgt[rows] + torch.randn((nd, V), generator=g, device=device) * draft_noise).to(dtype)
    tgt = tgt.to(dtype)
    if nd:
        ids = sample_from_probs(to_probs(drf, temperature, top_p, top_k), u=uniforms((nd,), g, device))
    else:
        ids = torch.zeros(0, dtype=torch.int64, device=device)
    return {
        "target": tgt, "draft": drf, "draft_ids": ids, "cu_k": cu.to(device), "k": k,
        "u_accept": uniforms((nd,), g, device), "u_final": uniforms((B,), g, device),
        "temperature": temperature, "top_p": top_p, "top_k": top_k,
    }


def greedy_inputs(B, k, V, seed, device, match=0.55, dtype=torch.bfloat16):
    """Greedy-verify workload: draft ids hit the target argmax w.p. `match`."""
    from .proposer_ops import greedy_draft_tokens
    g = torch.Generator(device=device).manual_seed(int(seed))
    tgt = zipf_logits(B * (k + 1), V, g, device, dtype=dtype).view(B, k + 1, V)
    am = greedy_draft_tokens(tgt[:, :k])
    other = (am + 1 + torch.randint(0, V - 1, (B, k), generator=g, device=device)) % V
    hit = torch.rand((B, k), generator=g, device=device) < match
    ids = torch.where(hit, am, other)
    return {"target": tgt, "draft_ids": ids, "u_accept": uniforms((B, k), g, device)}


def kv_inputs(layers, B, q, kv_heads, head_dim, block_size, len_lo, len_hi, seed, device,
              dtype=torch.bfloat16, alpha=0.6):
    """Paged-KV workload: lengths ~ U[len_lo, len_hi], a shuffled block table
    with room for q more positions, staged [L, 2, B, q, H*D] ~ N(0, 1), and a
    kept count per row in [0, q] from a geometric(alpha) truncated at q."""
    g = torch.Generator(device="cpu").manual_seed(int(seed))
    lengths = torch.randint(len_lo, len_hi + 1, (B,), generator=g)
    max_blocks = (len_hi + q + block_size - 1) // block_size
    num_blocks = B * max_blocks
    perm = torch.randperm(num_blocks, generator=g).to(torch.int32)
    block_table = perm.view(B, max_blocks)
    staged = torch.randn((layers, 2, B, q, kv_heads * head_dim), generator=g).to(dtype)
    # P(keep = a) proportional to alpha^a (1 - alpha), a = 0..q (truncated geometric)
    w = torch.tensor([alpha ** a * (1 - alpha) for a in range(q + 1)])
    keep = torch.multinomial(w / w.sum(), B, replacement=True, generator=g)
    return {
        "lengths": lengths.to(device), "block_table": block_table.to(device),
        "staged": staged.to(device), "keep": keep.to(device), "num_blocks": num_blocks,
        "max_blocks": max_blocks,
    }


def attn_inputs(B, seed, device, ctx_lo=1024, ctx_hi=8192, hq=32, hkv=8, d=128, block_size=16,
                alpha_lo=0.4, alpha_hi=0.9, c=0.1, k_max=8, dtype=torch.bfloat16):
    """Adaptive-k verify attention of one layer: row b drafts k_b = best_k(alpha_b, c)
    tokens (alpha_b ~ U(alpha_lo, alpha_hi)), so q_b = k_b + 1 new positions after
    a context of ctx_b ~ U[ctx_lo, ctx_hi] keys. K/V ~ N(0, 1) in a paged pool
    [num_blocks, block_size, hkv * d] behind a shuffled block table; q ~ N(0, 1)."""
    from .controller import best_k
    g = torch.Generator(device="cpu").manual_seed(int(seed))
    alphas = torch.rand(B, generator=g) * (alpha_hi - alpha_lo) + alpha_lo
    k = torch.tensor([best_k(float(a), c, k_max) for a in alphas], dtype=torch.int64)
    qb = k + 1
    ctx = torch.randint(ctx_lo, ctx_hi + 1, (B,), generator=g)
    kv_len = ctx + qb
    pages = (kv_len + block_size - 1) // block_size
    max_blocks = int(pages.max())
    num_blocks = int(pages.sum())
    perm = torch.randperm(num_blocks, generator=g).to(torch.int32)
    bt = torch.full((B, max_blocks), -1, dtype=torch.int32)
    o = 0
    for b in range(B):
        bt[b, :int(pages[b])] = perm[o:o + int(pages[b])]
        o += int(pages[b])
    cu_q = torch.zeros(B + 1, dtype=torch.int64)
    cu_q[1:] = torch.cumsum(qb, 0)
    gd = torch.Generator(device=device).manual_seed(int(seed) + 1)
    k_pool = torch.randn((num_blocks, block_size, hkv * d), generator=gd, device=device).to(dtype)
    v_pool = torch.randn((num_blocks, block_size, hkv * d), generator=gd, device=device).to(dtype)
    q = torch.randn((int(cu_q[-1]), hq, d), generator=gd, device=device).to(dtype)
    return {
        "q": q, "cu_q": cu_q.to(device), "k_pool": k_pool, "v_pool": v_pool,
        "block_table": bt.to(device), "kv_len": kv_len.to(device), "max_q": int(qb.max()),
        "k": k, "ctx": ctx, "hq": hq, "hkv": hkv, "d": d,
    }

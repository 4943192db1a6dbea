"""Seeded synthetic inputs of the verify-path workloads (no checkpoints, no data).

* verify:  B rows, k drafts, vocab V. Target logits ~ N(0, sigma^2) plus a Zipf
           boost `boost * rank^-s` on a seeded random permutation of the vocab
           per row; draft = target + N(0, draft_noise^2); draft ids drawn from
           the transformed draft distribution; fp32 uniforms for the accept
           test [B, k] and the final draw [B].
* greedy:  the same logits, draft ids equal to the target argmax with a given
           probability per position (else a different id).
* kv:      per-row lengths, a shuffled block table, staged K/V vectors.
"""
import torch

__all__ = ["zipf_logits", "uniforms", "verify_inputs", "greedy_inputs", "kv_inputs"]


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

"""Config 5 as one pipeline on the GPU: the per-row-k verify attention of a
target layer over paged KV, target logits projected from its output, then the
per-row-k sampler on those logits, with draft logits of the same positions plus
noise and draft ids drawn from them (bench/bench_engine.py:170-174 and
engine.py:273-303 at adaptive k).

Row b's attention rows [cu_q[b], cu_q[b+1]) are its k_b + 1 verify positions,
which is exactly where the sampler's packed layout keeps row b's target rows
(cu_k[b] + b onward), so the attention output feeds the sampler without
reordering. Checks: the attention output against the float64 oracle at bf16
tolerance (|gpu - oracle| <= 2e-2 + 2e-2 |oracle|) on sampled rows; n_acc, y
and flags bit for bit against the oracle sampler on the same logits.
"""
import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import sampling as O
from specdec.attention import verify_attention_paged
from specdec.sampling import rejection_sample_ragged, sample_from_probs, to_probs
from specdec.workloads import attn_inputs, uniforms

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_cfg5_attention_to_sampler_pipeline():
    B, V, T, tp, tk = 24, 151936, 0.7, 0.9, 50
    print(f"[cfg5 pipeline] B={B} V={V} contexts U[1024, 8192]", flush=True)
    inp = attn_inputs(B, seed=505, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    att = verify_attention_paged(inp["q"], inp["cu_q"], inp["k_pool"], inp["v_pool"],
                                 inp["block_table"], inp["kv_len"], inp["max_q"], error=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    cu_q = inp["cu_q"].cpu().numpy()
    kv = inp["kv_len"].cpu().numpy()
    d, bs = inp["d"], inp["k_pool"].shape[1]
    # the attention output on four rows (the longest context, the shortest, two others)
    g = np.random.default_rng(5)
    rows = sorted({int(kv.argmax()), int(kv.argmin()), *g.choice(B, 2, replace=False).tolist()})
    for b in rows:
        pages = (int(kv[b]) + bs - 1) // bs
        ids = inp["block_table"][b, :pages].long()
        q = inp["q"][int(cu_q[b]):int(cu_q[b + 1])].float().cpu().numpy()
        ref = OA.verify_attention_paged(q, np.array([0, q.shape[0]]),
                                        inp["k_pool"][ids].float().cpu().numpy(),
                                        inp["v_pool"][ids].float().cpu().numpy(),
                                        np.arange(pages)[None], kv[b:b + 1], 32, 8,
                                        1.0 / np.sqrt(d))
        got = att[int(cu_q[b]):int(cu_q[b + 1])].float().cpu().numpy()
        bad = np.abs(got - ref) > 2e-2 + 2e-2 * np.abs(ref)
        assert not bad.any(), (b, np.abs(got - ref).max())
    # target logits from the attention output: a seeded stand-in lm_head over its
    # first 512 features, scaled to logits of standard deviation 3
    nt = att.shape[0]
    gd = torch.Generator(device=DEV).manual_seed(506)
    w = torch.randn((512, V), generator=gd, device=DEV, dtype=torch.float32)
    h = att.reshape(nt, -1)[:, :512].float()
    tl = h @ w
    tl = tl * (3.0 / tl.std())
    # draft rows: the target logits of row b's drafted positions plus noise, ids
    # drawn from their to_probs
    k = [int(x) for x in inp["k"]]
    cu_k = torch.zeros(B + 1, dtype=torch.int64)
    cu_k[1:] = torch.cumsum(torch.tensor(k, dtype=torch.int64), 0)
    assert np.array_equal(cu_k.numpy() + np.arange(B + 1), cu_q)  # the shared packing
    nd = int(cu_k[-1])
    pos = torch.cat([torch.arange(int(cu_q[b]), int(cu_q[b]) + k[b]) for b in range(B)]).to(DEV)
    dl = (tl[pos] + torch.randn((nd, V), generator=gd, device=DEV)).to(torch.bfloat16)
    tl = tl.to(torch.bfloat16)
    draft_ids = sample_from_probs(to_probs(dl, T, tp, tk), u=uniforms((nd,), gd, DEV))
    ua, uf = uniforms((nd,), gd, DEV), uniforms((B,), gd, DEV)
    n, y, f = rejection_sample_ragged(tl, dl, draft_ids, ua, uf, cu_k.to(DEV), k_max=8,
                                      temperature=T, top_p=tp, top_k=tk)
    torch.cuda.synchronize()
    print(f"[cfg5 pipeline] {nt} target rows, {nd} draft rows: oracle", flush=True)
    f32 = lambda t: t.detach().float().cpu().numpy()
    rn, ry, rf = O.rejection_sample_ragged(f32(tl), f32(dl), draft_ids.cpu().numpy(), f32(ua),
                                           f32(uf), cu_k.numpy(), T, tp, tk)
    assert np.array_equal(n.cpu().numpy(), rn)
    assert np.array_equal(y.cpu().numpy(), ry)
    assert np.array_equal(f.cpu().numpy(), rf)

"""GPU parity of the MFMA verify attention (sdx_verify_attention_paged, head
dims 128 and 64) against the float64 oracle (oracle/attention.py), at bf16
tolerance: q, K and V are
bf16, the kernel accumulates in fp32 and rounds P (the softmax weights) and
the output to bf16, so |gpu - oracle| <= 2e-2 + 2e-2 |oracle| elementwise."""
import numpy as np
import pytest
import torch

from oracle import attention as OA
from specdec.attention import attention_workspace, verify_attention_paged
from specdec.workloads import attn_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check(inp, hq, hkv, atol=2e-2, rtol=2e-2, chunk_tokens=0):
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = verify_attention_paged(inp["q"], inp["cu_q"], inp["k_pool"], inp["v_pool"],
                                 inp["block_table"], inp["kv_len"], inp["max_q"], error=err,
                                 chunk_tokens=chunk_tokens)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    d = inp["q"].shape[-1]
    ref = OA.verify_attention_paged(inp["q"].float().cpu().numpy(), inp["cu_q"].cpu().numpy(),
                                    inp["k_pool"].float().cpu().numpy(),
                                    inp["v_pool"].float().cpu().numpy(),
                                    inp["block_table"].cpu().numpy(), inp["kv_len"].cpu().numpy(),
                                    hq, hkv, 1.0 / np.sqrt(d))
    got = out.float().cpu().numpy()
    bad = np.abs(got - ref) > atol + rtol * np.abs(ref)
    assert not bad.any(), (np.abs(got - ref).max(), np.argwhere(bad)[:5])
    return np.abs(got - ref).max()


@pytest.mark.parametrize("B,ctx_lo,ctx_hi,hq,hkv,k_max", [
    (6, 0, 40, 32, 8, 8),       # short contexts: tails inside the first tiles
    (5, 100, 300, 32, 8, 8),    # several tiles, ragged q_b from the controller
    (3, 2000, 2600, 8, 1, 8),   # group 8: up to 72 rows, two blocks of query rows
    (4, 37, 90, 16, 16, 3),     # no grouping (group 1)
])
def test_verify_attention_matches_oracle(B, ctx_lo, ctx_hi, hq, hkv, k_max):
    inp = attn_inputs(B, seed=B * 7 + ctx_lo, device=DEV, ctx_lo=ctx_lo, ctx_hi=ctx_hi, hq=hq,
                      hkv=hkv, k_max=k_max, alpha_lo=0.85, alpha_hi=0.95)
    _check(inp, hq, hkv)


@pytest.mark.parametrize("B,ctx_lo,ctx_hi,hq,hkv,k_max,chunk", [
    (6, 0, 40, 32, 8, 8, 0),          # short contexts
    (5, 100, 1500, 14, 2, 8, 128),    # 14 / 2 heads (group 7) over several chunks
    (4, 37, 90, 16, 16, 3, 0),        # no grouping
    (3, 2000, 2600, 32, 8, 8, 0),     # long rows, the library's chunking
])
def test_verify_attention_head_dim_64(B, ctx_lo, ctx_hi, hq, hkv, k_max, chunk):
    """Head dim 64 (the kernel's D = 64 instantiation: one K pass per tile, V
    held by half of each wave's lanes, four output column blocks)."""
    inp = attn_inputs(B, seed=B * 11 + ctx_lo, device=DEV, ctx_lo=ctx_lo, ctx_hi=ctx_hi, hq=hq,
                      hkv=hkv, d=64, k_max=k_max, alpha_lo=0.85, alpha_hi=0.95)
    _check(inp, hq, hkv, chunk_tokens=chunk)


@pytest.mark.parametrize("B,ctx_lo,ctx_hi,hq,hkv,d,k_max,chunk", [
    (4, 30, 200, 64, 8, 128, 8, 0),       # group 8, up to 72 rows: 2 row blocks, one chunk
    (3, 1500, 2600, 64, 8, 128, 8, 256),  # the same over several chunks
    (2, 100, 700, 32, 1, 128, 6, 128),    # group 32, up to 224 rows: 4 row blocks
    (3, 300, 900, 48, 2, 64, 8, 128),     # head dim 64, group 24, up to 216 rows
    (2, 4000, 4200, 64, 8, 128, 8, 64),   # 66 chunks x 72 rows: weights formed per element
])
def test_verify_attention_more_than_64_query_rows(B, ctx_lo, ctx_hi, hq, hkv, d, k_max, chunk):
    """A KV head with more than 64 query rows (q_b positions x query heads per
    KV head) gets a workgroup per block of 64 rows for each chunk; a row of
    several chunks is merged by the last of its chunks x blocks to finish."""
    inp = attn_inputs(B, seed=B * 13 + ctx_lo + hq, device=DEV, ctx_lo=ctx_lo, ctx_hi=ctx_hi,
                      hq=hq, hkv=hkv, d=d, k_max=k_max, alpha_lo=0.9, alpha_hi=0.97)
    assert inp["max_q"] * (hq // hkv) > 64
    _check(inp, hq, hkv, chunk_tokens=chunk)


def test_verify_attention_refuses_other_head_dims():
    from specdec._lib import SpecdecError
    inp = attn_inputs(2, seed=3, device=DEV, ctx_lo=10, ctx_hi=20, hq=8, hkv=2, d=96, k_max=3)
    with pytest.raises(SpecdecError):
        verify_attention_paged(inp["q"], inp["cu_q"], inp["k_pool"], inp["v_pool"],
                               inp["block_table"], inp["kv_len"], inp["max_q"])


@pytest.mark.parametrize("chunk", [64, 128, 1024])
def test_verify_attention_chunked_matches_oracle(chunk):
    """Rows split over several key chunks (merged from fp32 partials) and rows of
    one chunk, in one launch; the last chunk of a row may hold no key that a
    query row sees (fully masked partial)."""
    inp = attn_inputs(6, seed=chunk, device=DEV, ctx_lo=1, ctx_hi=1500, hq=32, hkv=8, k_max=8,
                      alpha_lo=0.85, alpha_hi=0.95)
    _check(inp, 32, 8, chunk_tokens=chunk)


@pytest.mark.parametrize("bs,chunk", [(1, 1024), (12, 128), (16, 64)])
def test_verify_attention_block_sizes(bs, chunk):
    """Pages of 1 token (a page id per token), 12 tokens (page boundaries
    inside tiles, general index arithmetic) and 16, with long rows."""
    inp = attn_inputs(2, seed=bs, device=DEV, ctx_lo=1500, ctx_hi=2600, hq=8, hkv=2, k_max=6,
                      block_size=bs)
    _check(inp, 8, 2, chunk_tokens=chunk)


@pytest.mark.parametrize("seed", range(6))
def test_verify_attention_random_shapes(seed):
    """Seeded random shapes: batch, query/KV heads (group 1 to 8), k_max within
    the 64-row limit, context range, block size and chunk size."""
    rng = np.random.RandomState(100 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 4, 8]))
    hq = hkv * group
    k_max = int(min(8, 64 // group - 1))
    lo = int(rng.randint(0, 1500))
    hi = lo + int(rng.randint(1, 1500))
    bs = int(rng.choice([1, 3, 8, 16, 32]))
    chunk = int(rng.choice([0, 64, 192, 512]))
    B = int(rng.randint(1, 7))
    inp = attn_inputs(B, seed=seed, device=DEV, ctx_lo=lo, ctx_hi=hi, hq=hq, hkv=hkv, k_max=k_max,
                      block_size=bs, alpha_lo=0.5, alpha_hi=0.95)
    _check(inp, hq, hkv, chunk_tokens=chunk)


def test_verify_attention_same_for_any_chunking():
    inp = attn_inputs(4, seed=11, device=DEV, ctx_lo=300, ctx_hi=900, hq=16, hkv=4, k_max=6)
    outs = [verify_attention_paged(inp["q"], inp["cu_q"], inp["k_pool"], inp["v_pool"],
                                   inp["block_table"], inp["kv_len"], inp["max_q"],
                                   chunk_tokens=ch).float() for ch in (64, 192, 1024)]
    for o in outs[1:]:
        # rounding of P to bf16 is relative to each chunk's running max
        assert torch.allclose(o, outs[0], atol=1e-2, rtol=1e-2)


def test_verify_attention_rejects_bad_rows():
    inp = attn_inputs(3, seed=5, device=DEV, ctx_lo=20, ctx_hi=40, hq=8, hkv=2, k_max=4)
    bt = inp["block_table"].clone()
    bt[1, 0] = 10 ** 6                      # a page id outside the pool
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    verify_attention_paged(inp["q"], inp["cu_q"], inp["k_pool"], inp["v_pool"], bt,
                           inp["kv_len"], inp["max_q"], error=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 1
    with pytest.raises(RuntimeError):       # chunk not a multiple of 64
        verify_attention_paged(inp["q"], inp["cu_q"], inp["k_pool"], inp["v_pool"],
                               inp["block_table"], inp["kv_len"], inp["max_q"], chunk_tokens=96)


def test_verify_attention_graph_replays():
    """The call captured in a graph (plan and attention kernels; no memsets): every
    replay, with eager calls and synchronizations between replays, equals the
    eager output bit for bit (the kernels are deterministic)."""
    hq, hkv = 32, 8
    inp = attn_inputs(8, seed=31, device=DEV, ctx_lo=500, ctx_hi=3000, hq=hq, hkv=hkv, k_max=8,
                      alpha_lo=0.85, alpha_hi=0.95)
    args = (inp["q"], inp["cu_q"], inp["k_pool"], inp["v_pool"], inp["block_table"],
            inp["kv_len"], inp["max_q"])
    eager = verify_attention_paged(*args).clone()
    torch.cuda.synchronize()
    _check(inp, hq, hkv)
    B = inp["cu_q"].numel() - 1
    ws = attention_workspace(B, inp["max_q"], hq, hkv, inp["k_pool"].shape[1],
                             inp["block_table"].shape[1], device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.empty_like(inp["q"])
    verify_attention_paged(*args, out=out, error=err, workspace=ws)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        verify_attention_paged(*args, out=out, error=err, workspace=ws)
    for _ in range(5):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert torch.equal(verify_attention_paged(*args), eager)  # eager work between replays
        torch.cuda.synchronize()
    assert int(err.item()) == 0


def test_verify_attention_long_rows_unstaged_merge():
    """Chunks of 64 keys over contexts near 8192 with 9 query positions x group 4
    (36 rows per KV head): 128 chunks x 36 rows = 4608 chunk weights, more than
    the 2112 the merging workgroup's tile buffers hold at head dim 128, so the
    merge forms its weights per element instead of staging them in LDS."""
    inp = attn_inputs(2, seed=64, device=DEV, ctx_lo=8000, ctx_hi=8192, hq=32, hkv=8, k_max=8,
                      alpha_lo=0.97, alpha_hi=0.99)
    nch = (int(inp["kv_len"].max()) + 63) // 64
    assert nch * inp["max_q"] * 4 > 2112
    _check(inp, 32, 8, chunk_tokens=64)


def test_verify_attention_bench_shape_sampled_rows():
    """The bench shape: B=128 rows of contexts U[1024, 8192], k_b from the
    controller's best_k (alpha ~ U(0.4, 0.9), k_max 8), 32/8 heads x 128, block
    16, the library's default chunking, in one launch. Eight rows (the longest,
    the shortest and six others) are checked against the float64 oracle, each
    on its own pages."""
    inp = attn_inputs(128, seed=2024, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = verify_attention_paged(inp["q"], inp["cu_q"], inp["k_pool"], inp["v_pool"],
                                 inp["block_table"], inp["kv_len"], inp["max_q"], error=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    kv = inp["kv_len"].cpu().numpy()
    cu = inp["cu_q"].cpu().numpy()
    g = np.random.default_rng(7)
    rows = sorted({int(kv.argmax()), int(kv.argmin()), *g.choice(128, 6, replace=False).tolist()})
    d, bs = inp["d"], inp["k_pool"].shape[1]
    for b in rows:
        pages = (int(kv[b]) + bs - 1) // bs
        ids = inp["block_table"][b, :pages].long()
        kp = inp["k_pool"][ids].float().cpu().numpy()
        vp = inp["v_pool"][ids].float().cpu().numpy()
        q = inp["q"][int(cu[b]):int(cu[b + 1])].float().cpu().numpy()
        ref = OA.verify_attention_paged(q, np.array([0, q.shape[0]]), kp, vp,
                                        np.arange(pages)[None], kv[b:b + 1], 32, 8,
                                        1.0 / np.sqrt(d))
        got = out[int(cu[b]):int(cu[b + 1])].float().cpu().numpy()
        bad = np.abs(got - ref) > 2e-2 + 2e-2 * np.abs(ref)
        assert not bad.any(), (b, np.abs(got - ref).max())

"""The two-launch form of the bf16 verify (row statistics, then the draw) and of
the bf16 draft step (row statistics, the draw, then the epilogue kernel)
against the one-launch kernels that replace them by default.

SDX_VERIFY_FUSED=0 selects the two-launch forms once per process, so a child
process computes the same seeded cases with them and the outputs (n_acc, y,
flags; x, q(x), conf, stop) must equal this process's one-launch outputs bit
for bit. The uniform verify case and the draft step are also checked against
the oracle here, so both forms are pinned to it directly.
"""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
HERE = os.path.dirname(os.path.abspath(__file__))


def run_cases():
    """n_acc, y and flags of each case, as numpy arrays keyed by case name."""
    from specdec import sampling as S
    from specdec.workloads import ragged_verify_inputs, uniforms, verify_inputs, zipf_logits
    out = {}
    # one k per batch row: B=64 k=4 at V=151936 (rows past the CU multiple are split)
    inp = verify_inputs(64, 4, 151936, seed=31, device=DEV)
    r = S.rejection_sample(inp["target"], inp["draft"], inp["draft_ids"], inp["u_accept"],
                           inp["u_final"], temperature=0.8, top_p=0.95)
    for name, t in zip(("n", "y", "f"), r):
        out[f"uniform_{name}"] = t.cpu().numpy()
    # per-row k, config 5's sampler with inactive rows
    B = 40
    inp = ragged_verify_inputs(B, 151936, seed=32, device=DEV)
    active = torch.tensor([b % 7 != 3 for b in range(B)], device=DEV)
    r = S.rejection_sample_ragged(inp["target"], inp["draft"], inp["draft_ids"], inp["u_accept"],
                                  inp["u_final"], inp["cu_k"], temperature=0.7, top_p=0.9,
                                  top_k=50, active=active)
    for name, t in zip(("n", "y", "f"), r):
        out[f"ragged_{name}"] = t.cpu().numpy()
    # per-row k from 0 to 8 at a small vocabulary
    ks = [3, 0, 8, 1, 5, 2, 8, 4, 0, 6, 7, 2]
    inp = ragged_verify_inputs(len(ks), 4096, seed=33, device=DEV, temperature=1.0, top_p=1.0,
                               top_k=0, k=ks)
    r = S.rejection_sample_ragged(inp["target"], inp["draft"], inp["draft_ids"], inp["u_accept"],
                                  inp["u_final"], inp["cu_k"], k_max=8, temperature=1.0,
                                  top_p=1.0, top_k=0)
    for name, t in zip(("n", "y", "f"), r):
        out[f"ragged_small_{name}"] = t.cpu().numpy()
    # the draft step, B=64 at V=151936 with conf and the early-exit flag
    g = torch.Generator(device=DEV).manual_seed(34)
    x = zipf_logits(64, 151936, g, DEV)
    u = uniforms((64,), g, DEV)
    conf = 0.3 + 0.7 * uniforms((64,), g, DEV)
    xs, qx, stop = S.draft_step(x, u, 0.8, 0.95, 0, conf=conf, tau=0.5, step=2, min_k=1)
    out["draft_x"], out["draft_qx"] = xs.cpu().numpy(), qx.cpu().numpy()
    out["draft_conf"], out["draft_stop"] = conf.cpu().numpy(), stop.cpu().numpy()
    return out


def test_two_launch_form_equals_fused(tmp_path):
    dst = tmp_path / "two_launch.npz"
    child = (f"import sys; sys.path[:0] = [{HERE!r}, {os.path.dirname(HERE)!r}, "
             f"{os.path.join(os.path.dirname(HERE), 'adaptive-specdec_amd')!r}]\n"
             "import numpy as np, test_gpu_two_launch as T\n"
             f"np.savez({str(dst)!r}, **T.run_cases())\n")
    env = dict(os.environ, SDX_VERIFY_FUSED="0")
    print("two-launch child process: uniform B=64 k=4, ragged B=40 and B=12", flush=True)
    subprocess.run([sys.executable, "-c", child], env=env, check=True, timeout=300)
    two = np.load(dst)
    fused = run_cases()
    assert sorted(two.files) == sorted(fused)
    for key, got in fused.items():
        assert np.array_equal(two[key], got), key
    # ... and the oracle on the same inputs (the generators replay the cases)
    from oracle import sampling as O
    from specdec.workloads import uniforms, verify_inputs, zipf_logits
    f32 = lambda t: t.detach().float().cpu().numpy()
    inp = verify_inputs(64, 4, 151936, seed=31, device=DEV)
    rn, ry, rf = O.rejection_sample(f32(inp["target"]), f32(inp["draft"]),
                                    inp["draft_ids"].cpu().numpy(), f32(inp["u_accept"]),
                                    f32(inp["u_final"]), 0.8, 0.95, 0)
    assert np.array_equal(fused["uniform_n"], rn) and np.array_equal(fused["uniform_y"], ry)
    assert np.array_equal(fused["uniform_f"], rf)
    g = torch.Generator(device=DEV).manual_seed(34)
    x = zipf_logits(64, 151936, g, DEV)
    u = uniforms((64,), g, DEV)
    conf0 = 0.3 + 0.7 * uniforms((64,), g, DEV)
    rx, rq, rc, rs = O.draft_step(f32(x), f32(u), 0.8, 0.95, 0, conf=f32(conf0), tau=0.5, step=2,
                                  min_k=1)
    assert np.array_equal(fused["draft_x"], rx)
    assert np.array_equal(fused["draft_qx"].view(np.uint32), rq.view(np.uint32))
    assert np.array_equal(fused["draft_conf"].view(np.uint32), rc.view(np.uint32))
    assert int(fused["draft_stop"][0]) == rs

"""The two-launch form of the bf16 verify (row statistics, then the draw) against
the fused kernel that replaces it by default.

SDX_VERIFY_FUSED=0 selects the two-launch form once per process, so a child
process computes the same seeded cases with it and the outputs (n_acc, y,
flags) must equal this process's fused outputs bit for bit. The fused outputs
are checked against the oracle by test_gpu_sampling.py.
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
    from specdec.workloads import ragged_verify_inputs, verify_inputs
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

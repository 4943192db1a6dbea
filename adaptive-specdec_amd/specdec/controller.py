"""Closed-form draft length (`specdec/controller.py:47-67`), host side.

The expected tokens per round of Leviathan et al., (1 - a^(k+1)) / (1 - a),
over the cost of the round in target forwards, (k + x) c + 1, where x is the
number of draft forwards a round costs beyond k (1 for the from-scratch engine,
0 for the vLLM proposer, `vllm_draft_spec/proposer.py:89`). The verify path
uses it to pick a per-row k.

`DeviceController` keeps the EWMAAnalytic state (`controller.py:121-154`) on
the device and updates it from the verify's device n_acc, so choosing the next
k needs no host round trip.
"""
import numpy as np
import torch

from . import _lib

__all__ = ["expected_speedup", "best_k", "best_k_rows", "DeviceController"]


def expected_speedup(k, alpha, c, extra_fwd=1):
    """Expected tokens per round divided by the round's cost (`controller.py:47-61`)."""
    k = max(1, int(k))
    if alpha >= 1.0 - 1e-9:
        tokens = float(k + 1)
    else:
        tokens = (1.0 - alpha ** (k + 1)) / (1.0 - alpha)
    return tokens / ((k + extra_fwd) * c + 1.0)


def best_k(alpha, c, k_max=8, extra_fwd=1):
    """argmax over k in [1, k_max] (`controller.py:64-67`); the smallest k wins ties."""
    return max(range(1, int(k_max) + 1), key=lambda k: expected_speedup(k, alpha, c, extra_fwd))


def best_k_rows(alphas, c, k_max=8, extra_fwd=1):
    """best_k for each row's acceptance estimate (a list of per-row k)."""
    return [best_k(float(a), c, k_max, extra_fwd) for a in alphas]


class DeviceController:
    """EWMAAnalytic (`controller.py:121-154`) with its state on the device.

    mode "batch": one controller for the whole batch, exactly the reference's
    (accepted = sum n_acc, reached = sum min(n_acc + 1, k)); mode "row": one per
    batch row (each row's own acceptance estimate and k, the offsets cu_k of the
    next per-row-k verify produced on the device). `update(n_acc, k_used)`
    queues one kernel; `k` / `cu_k` are device tensors holding the next round's
    choice. The float64 state follows the host controller's formulas.
    """

    def __init__(self, batch, mode="batch", k_max=8, beta=0.99, k_init=4, c_init=0.15, warmup=3,
                 extra_fwd=1, device="cuda"):
        if mode not in ("batch", "row"):
            raise ValueError(f"unknown controller mode {mode!r}")
        self.B, self.mode = int(batch), mode
        self.k_max, self.beta, self.k_init = int(k_max), float(beta), int(k_init)
        self.warmup, self.extra_fwd = int(warmup), int(extra_fwd)
        n = 1 if mode == "batch" else self.B
        dev = torch.device(device)
        # sdx_ctrl_state: acc, reached, c (float64), rounds, last_k (int32) = 4 doubles
        st = torch.zeros((n, 4), dtype=torch.float64)
        st[:, 2] = float(c_init)
        last = torch.tensor([0, self.k_init], dtype=torch.int32).view(torch.float64)
        st[:, 3] = last
        self.state = st.to(dev)
        self.k = torch.full((n,), self.k_init, dtype=torch.int64, device=dev)
        self._k_next = torch.empty_like(self.k)
        self.cu_k = None
        if mode == "row":
            self.cu_k = (torch.arange(self.B + 1, dtype=torch.int64) * self.k_init).to(dev)

    def update(self, n_acc, k_used=None, c_obs=None):
        """One round's n_acc [B] (device int64) drafted at k_used ([1] for the batch
        mode, [B] per row; default: the k this controller proposed). c_obs: the
        observed draft/target forward-time ratio ([1] fp32 device tensor), or None
        to keep c. Updates the state and `k` (and `cu_k`) in place on the device."""
        _lib.require_gpu(n_acc)
        n_acc = n_acc.to(torch.int64).contiguous()
        ku = (self.k if k_used is None else k_used.to(torch.int64)).contiguous()
        k_next = self._k_next
        rc = _lib.lib().sdx_controller_update(
            _lib.ptr(self.state), self.state.shape[0], _lib.ptr(n_acc), self.B, _lib.ptr(ku),
            self.beta, self.k_max, self.k_init, self.warmup, self.extra_fwd, _lib.ptr(c_obs),
            _lib.ptr(k_next), _lib.ptr(self.cu_k), _lib.stream_of(n_acc))
        _lib.check(rc, "DeviceController.update")
        self.k.copy_(k_next)
        return self.k

    def host_state(self):
        """(acc, reached, c, rounds, last_k) per state, read back (one sync)."""
        st = self.state.cpu().numpy()
        ints = np.ascontiguousarray(st[:, 3]).view(np.int32).reshape(-1, 2)
        return [(float(r[0]), float(r[1]), float(r[2]), int(i[0]), int(i[1]))
                for r, i in zip(st, ints)]

"""ctypes binding of libspecdec_amd.so (the C ABI in include/specdec_amd.h).

The library is built in-tree by `adaptive-specdec_amd/build.py` (or
`__graft_entry__.build()`). There is no fallback: if it is missing, or a tensor
is not on a ROCm device, calls raise.
"""
import ctypes
import os

import torch

_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libspecdec_amd.so")
_LIB = None

F32, BF16, F16 = 0, 1, 2
_DTYPE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}
# Longest fp16 row the library's fp16 kernels take (their row kernel holds a row
# in registers). The Python entry points widen longer fp16 rows to fp32, which
# is exact, and run the fp32 kernels (rows up to 262,144).
F16_MAX_VOCAB = 163840


def widen_f16(x):
    """fp16 rows longer than F16_MAX_VOCAB as fp32 (exact); anything else as is."""
    return x.float() if x.dtype == torch.float16 and x.shape[-1] > F16_MAX_VOCAB else x

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int32
F = ctypes.c_float
D = ctypes.c_double
SZ = ctypes.c_size_t
INT = ctypes.c_int

# name -> (restype, argtypes)
_SIGS = {
    "sdx_last_error": (ctypes.c_char_p, []),
    "sdx_version": (INT, []),
    "sdx_workspace_init": (INT, [P, SZ, P]),
    "sdx_to_probs_workspace": (SZ, [I64, I64, INT]),
    "sdx_to_probs": (INT, [P, INT, I64, I64, I64, F, F, I32, P, I64, P, SZ, P]),
    "sdx_sample_probs_workspace": (SZ, [I64, I64]),
    "sdx_sample_probs": (INT, [P, I64, I64, I64, P, P, P, SZ, P]),
    "sdx_residual_probs_workspace": (SZ, [I64, I64]),
    "sdx_residual_probs": (INT, [P, P, I64, I64, I64, P, I64, P, SZ, P]),
    "sdx_gather_prob": (INT, [P, I64, I64, I64, P, P, P]),
    "sdx_verify_workspace": (SZ, [I64, I32, I64, INT]),
    "sdx_verify": (INT, [P, P, INT, I64, I32, I64, P, P, P, P, F, F, I32, P, P, P, P, SZ, P]),
    "sdx_verify_noalloc": (INT, [P, P, INT, I64, I32, I64, P, P, P, P, F, F, I32, P, P, P, P]),
    "sdx_verify_ragged_workspace": (SZ, [I64, I64, I64, INT]),
    "sdx_verify_ragged": (INT, [P, P, INT, I64, I32, I64, I64, P, P, P, P, P, F, F, I32, P, P, P, P,
                                SZ, P]),
    "sdx_verify_drafted": (INT, [P, P, INT, I64, I32, I64, P, P, P, P, F, F, I32, P, P, P, P, P,
                                 SZ, P]),
    "sdx_verify_counter_layout": (INT, [I64, I64, I32, I64, INT, I32, P, I32]),
    "sdx_verify_stats": (INT, [P, P, INT, I64, I32, I64, P, F, F, I32, P, SZ, P]),
    "sdx_verify_greedy_workspace": (SZ, [I64, I32]),
    "sdx_verify_greedy": (INT, [P, INT, I64, I32, I64, P, P, P, P, P, P, P, SZ, P]),
    "sdx_draft_step_workspace": (SZ, [I64, I64, INT]),
    "sdx_draft_step": (INT, [P, INT, I64, I64, I64, F, F, I32, P, P, P, P, F, I32, I32, P, P, SZ,
                             P]),
    "sdx_round_commit": (INT, [I64, I32, P, P, P, P, P, P, P, I64, P, I32, P, P, P, P, P, P]),
    "sdx_controller_update": (INT, [P, I64, P, I64, P, D, I32, I32, I32, I32, P, P, P, P]),
    "sdx_argmax": (INT, [P, INT, I64, I64, I64, P, P]),
    "sdx_slot_mapping": (INT, [P, I64, I64, P, I32, I64, I64, P, P, P]),
    "sdx_kv_advance": (INT, [P, I64, I64, P]),
    "sdx_kv_rollback": (INT, [P, I64, P, P, P]),
    "sdx_ragged_update": (INT, [P, P, P, P, INT, I64, I64, I64, I64, I64, P, P, P]),
    "sdx_attn_mask": (INT, [P, P, I64, I64, I64, F, INT, P, P]),
    "sdx_kv_append_paged": (INT, [P, I64, I64, P, INT, I32, I64, I64, I64, P, I64, I32, I64, P,
                                  P, P]),
    "sdx_verify_attention_paged": (INT, [P, INT, I64, P, I32, I32, I32, I32, P, P, I64, I32, P,
                                         I64, P, F, I32, P, SZ, P, P, P]),
    "sdx_verify_attention_workspace": (SZ, [I64, I32, I32, I32, I32, I64, I32]),
}

EXPORTS = tuple(_SIGS)


class SpecdecError(RuntimeError):
    """A libspecdec_amd call returned an error status."""


def library_path():
    return _PATH


def lib():
    """Load (once) and return the ctypes library with typed entry points."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(_PATH):
            raise ImportError(
                f"{_PATH} is not built; run `python adaptive-specdec_amd/build.py` "
                "(hipcc, gfx950) before using specdec")
        L = ctypes.CDLL(_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(rc, what):
    if rc != 0:
        msg = lib().sdx_last_error().decode(errors="replace")
        raise SpecdecError(f"{what} failed ({rc}): {msg}")


def dtype_code(t):
    try:
        return _DTYPE[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32, bfloat16 or float16")


def require_gpu(*tensors):
    """Every tensor must live on the ROCm device; there is no CPU path."""
    for t in tensors:
        if t is not None and (not isinstance(t, torch.Tensor) or t.device.type != "cuda"):
            raise RuntimeError(
                "specdec (MI355X build) runs on ROCm device tensors only; got "
                f"{getattr(t, 'device', type(t))}")


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def workspace(nbytes, device, prepare=True):
    """A new workspace of at least `nbytes`; with `prepare`, prepared by
    sdx_workspace_init on the current stream (zero-filled, header word set: the
    verify entry points keep arrival counters in it that every call leaves at
    zero)."""
    n = (max(int(nbytes), 1) + 255) // 256 * 256
    ws = torch.empty(n, dtype=torch.uint8, device=device)
    if prepare:
        check(lib().sdx_workspace_init(ptr(ws), n, stream_of(ws)), "sdx_workspace_init")
    return ws


_WS_CACHE = {}
# entry points whose workspace must be prepared (they keep arrival counters or
# per-row state in it); the others use theirs as plain scratch
_PREPARED_KINDS = {"verify", "draft", "greedy"}


def cached_workspace(nbytes, device, kind):
    """The current stream's reusable workspace for entry points of one `kind`,
    grown when too small. Calls queued on one stream run in order, so they may
    share it; each stream has its own. Kinds never share memory: the verify
    workspaces keep their header (magic word and zeroed counters) at fixed
    offsets that other entry points would overwrite. Under graph capture a new
    workspace is allocated (from the graph's pool) and not kept."""
    dev = torch.device(device)
    prepare = kind in _PREPARED_KINDS
    if torch.cuda.is_current_stream_capturing():
        return workspace(nbytes, dev, prepare)
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream, kind)
    ws = _WS_CACHE.get(key)
    if ws is None or ws.numel() < int(nbytes):
        ws = workspace(nbytes, dev, prepare)
        _WS_CACHE[key] = ws
    return ws


def prepare(ws):
    """Prepare an existing workspace again (sdx_workspace_init on the current
    stream): needed after a verify call flagged rows SDX_FLAG_WORKSPACE because a
    draw's bounded wait gave up, which marks the workspace header."""
    check(lib().sdx_workspace_init(ptr(ws), ws.numel(), stream_of(ws)), "sdx_workspace_init")


def reset_workspaces():
    """Prepare every cached workspace of the prepared kinds again (see `prepare`)."""
    for (_, _, kind), ws in _WS_CACHE.items():
        if kind in _PREPARED_KINDS:
            prepare(ws)

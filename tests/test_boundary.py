"""CPU checks of the C-ABI boundary and the host-side logic (no GPU needed).

* libspecdec_amd.so loads and exports every function include/specdec_amd.h declares;
* the ctypes signature table covers exactly that set;
* the Python entry points refuse CPU tensors (there is no CPU fallback);
* host logic: controller closed form, RaggedCache host bookkeeping errors;
* argument checks of the C ABI, which return their status before any HIP work.
"""
import ctypes
import os
import re

import pytest
import torch

from conftest import REPO

HEADER = os.path.join(REPO, "include", "specdec_amd.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(sdx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert "sdx_verify" in names and "sdx_to_probs" in names and "sdx_kv_rollback" in names


def test_library_exports_every_declared_symbol():
    from specdec import _lib
    path = _lib.library_path()
    if not os.path.exists(path):
        pytest.skip("libspecdec_amd.so not built (run __graft_entry__.build())")
    so = ctypes.CDLL(path)
    missing = [n for n in declared() if not hasattr(so, n)]
    assert not missing, missing
    assert sorted(_lib.EXPORTS) == declared()
    L = _lib.lib()
    assert L.sdx_version() >= 1
    # workspace queries are pure host arithmetic
    assert L.sdx_verify_workspace(64, 4, 151936, _lib.BF16) > 64 * 9 * 64
    assert L.sdx_to_probs_workspace(8, 151936, _lib.BF16) > 0


def test_python_api_refuses_cpu_tensors():
    from specdec import sampling
    x = torch.zeros(2, 16)
    with pytest.raises(RuntimeError, match="ROCm device"):
        sampling.to_probs(x)
    with pytest.raises(RuntimeError, match="ROCm device"):
        sampling.rejection_sample(torch.zeros(1, 2, 16), torch.zeros(1, 1, 16),
                                  torch.zeros(1, 1, dtype=torch.long), torch.zeros(1, 1),
                                  torch.zeros(1))


def test_controller_matches_oracle():
    from oracle import controller as OC
    from specdec import controller as C
    for a in (0.1, 0.4, 0.55, 0.7, 0.9, 0.99, 1.0):
        for c in (0.05, 0.1, 0.3, 1.6):
            for x in (0, 1):
                assert C.best_k(a, c, 8, x) == OC.best_k(a, c, 8, x)
                assert C.expected_speedup(4, a, c, x) == OC.expected_speedup(4, a, c, x)
    assert C.best_k_rows([0.4, 0.9], 0.1) == [C.best_k(0.4, 0.1), C.best_k(0.9, 0.1)]


def test_ragged_cache_host_bookkeeping():
    """Host half of `kvcache.py:165-202` (no kernel calls): lengths, max_len,
    uniformity, positions and the below-zero error, on a CPU-placed cache."""
    from specdec.kvcache import RaggedCache
    c = RaggedCache(3, 3, 128, "cpu")
    assert c.batch_size == 3 and len(c.layers) == 3 and c.get_seq_length() == 0
    c.set_lengths(torch.tensor([7, 5, 6]))
    assert (c.max_len, c._uniform) == (7, False)
    c.advance(4)
    c.rollback([0, 3, 2])
    assert c.lengths.tolist() == [11, 6, 8] and c.max_len == 11
    assert c.positions(2).tolist() == [[11, 12], [6, 7], [8, 9]]
    assert c.cache_position(2).tolist() == [11, 12]
    assert c.kv_len_for(3) == 14
    with pytest.raises(RuntimeError, match="below zero"):
        c.rollback(torch.tensor([12, 0, 0]))
    c2 = RaggedCache(1, 2, 16, "cpu")
    c2.set_lengths([4, 4])
    assert c2.attn_mask(2, torch.float32) is None          # uniform, no pad: no mask


def test_c_abi_argument_errors():
    """Status codes of the argument checks: a workspace one byte short, a vocab
    past the 16-bit row kernel's capacity, an unsupported head size and a bad
    chunk size fail with SDX_EWORKSPACE / SDX_EUNSUPPORTED / SDX_EINVAL and a
    message, before anything is launched (the pointers are never dereferenced)."""
    from specdec import _lib
    L = _lib.lib()
    OK, EINVAL, EUNSUP, EWS = 0, -1, -2, -4
    BF16 = 1
    fake = ctypes.c_void_p(4096)
    B, k, V = 4, 2, 1024
    need = L.sdx_verify_workspace(B, k, V, BF16)
    assert need > 0

    def verify(batch, kk, vocab, ws_bytes, draft_ids=fake):
        return L.sdx_verify(fake, fake, BF16, batch, kk, vocab, draft_ids, fake, fake, None,
                            ctypes.c_float(0.8), ctypes.c_float(0.95), 0, fake, fake, fake,
                            fake, ws_bytes, None)

    assert verify(B, k, V, need - 1) == EWS
    assert b"workspace" in L.sdx_last_error()
    assert verify(B, k, (1 << 18), 1 << 40) == EUNSUP  # bf16 rows: vocab <= 2^18 - 8
    assert b"vocab" in L.sdx_last_error()
    F16 = 2
    assert L.sdx_to_probs(fake, F16, 1, 163840 + 8, 163840 + 8, ctypes.c_float(0.8),
                          ctypes.c_float(0.95), 0, fake, 163840 + 8, fake, 1 << 40, None) == EUNSUP
    # fp32 to_probs: the output rows may not overlap the logits (in place is refused)
    F32 = 0
    Vf = 151936
    assert L.sdx_to_probs(fake, F32, 2, Vf, Vf, ctypes.c_float(0.8), ctypes.c_float(0.95), 0,
                          ctypes.c_void_p(4096 + 4 * Vf), Vf, fake, 1 << 40, None) == EINVAL
    assert b"overlap" in L.sdx_last_error()
    assert verify(B, 0, V, need) == EINVAL
    assert verify(B, k, V, need, draft_ids=None) == EINVAL
    assert verify(0, k, V, need) == OK  # an empty batch is a no-op
    # verify attention: chunk sizes are 0 or multiples of 64 up to 1024; head_dim 64 or 128
    assert L.sdx_verify_attention_workspace(8, 5, 32, 8, 16, 64, 96) == 0
    assert L.sdx_verify_attention_workspace(8, 5, 32, 8, 16, 64, 0) > 0
    rc = L.sdx_verify_attention_paged(fake, BF16, 8, fake, 5, 32, 8, 96, fake, fake, 100, 16,
                                      fake, 64, fake, ctypes.c_float(0.125), 0, fake, 1 << 30,
                                      fake, None, None)
    assert rc == EUNSUP and b"head_dim" in L.sdx_last_error()
    # round commit: drafted ids are required whenever a row may have drafted
    i64 = ctypes.c_void_p(8192)

    def commit(kk, cu, ids):
        return L.sdx_round_commit(4, kk, cu, i64, i64, ids, fake, i64, i64, 8, None, 0, None,
                                  None, None, None, None, None)

    assert commit(2, None, None) == EINVAL
    assert commit(0, i64, None) == EINVAL       # per-row k: any row may draft


def test_verify_counters_lie_in_the_header():
    """Every cross-workgroup counter the verify launches are handed (split-row
    arrivals, the fused kernel's row arrivals and draw counters) lies inside the
    fixed 16 KB header, after the magic word, and the ranges do not overlap, for
    every shape the entry points accept (one k and per-row k, bf16 / fp16 / fp32,
    devices of 1 to 304 compute units). A counter carved anywhere else would be
    found stale by a later call of another shape."""
    from specdec import _lib
    L = _lib.lib()
    HDR = 16384
    r = (ctypes.c_int64 * 8)()
    shapes = [(1, 1), (4, 4), (64, 4), (256, 8), (1024, 4), (300, 31), (1000, 2), (2048, 4),
              (64, 40)]
    n_checked = 0
    for dt in (0, 1, 2):
        for V in (16, 1000, 32000, 151936, 262136):
            for B, k in shapes:
                for ragged in (False, True):
                    for cus in (1, 8, 80, 256, 304):
                        tr = B * (k + 1) - (B // 3 if ragged else 0) if ragged else 0
                        n = L.sdx_verify_counter_layout(B, tr, k, V, dt, cus, r, 4)
                        assert n == 4, (dt, V, B, k, cus)
                        rng = [(r[2 * i], r[2 * i + 1]) for i in range(n)]
                        h0, h1 = rng[-1]
                        assert (h0, h1) == (0, HDR)
                        used = [(b, e) for b, e in rng[:-1] if e > b]
                        for b, e in used:
                            assert 4 <= b <= e <= HDR, (dt, V, B, k, cus, b, e)
                        used.sort()
                        for (b0, e0), (b1, _) in zip(used, used[1:]):
                            assert e0 <= b1, (dt, V, B, k, cus, used)
                        n_checked += 1
    assert n_checked > 1000


def test_long_fp16_rows_are_widened_for_the_fp32_kernels():
    """The Python entry points hand fp16 rows longer than the fp16 kernels take
    (F16_MAX_VOCAB, the C ABI's fp16 limit) to the fp32 kernels, widened
    exactly; every other row goes to the kernels as it is."""
    from specdec import _lib
    L = _lib.lib()
    fake = ctypes.c_void_p(16)
    EUNSUP = -2  # SDX_EUNSUPPORTED
    # the C ABI's limit is the one the Python layer widens past
    assert L.sdx_to_probs(fake, _lib.F16, 1, _lib.F16_MAX_VOCAB + 8, _lib.F16_MAX_VOCAB + 8,
                          ctypes.c_float(0.8), ctypes.c_float(0.95), 0, fake,
                          _lib.F16_MAX_VOCAB + 8, fake, 1 << 40, None) == EUNSUP
    x = (torch.arange(2 * (_lib.F16_MAX_VOCAB + 8)) % 2000 - 1000).reshape(2, -1).to(torch.float16)
    w = _lib.widen_f16(x)
    assert w.dtype == torch.float32 and torch.equal(w, x.float())
    for t in (x[:, :_lib.F16_MAX_VOCAB], x.to(torch.bfloat16), x.float()):
        assert _lib.widen_f16(t) is t

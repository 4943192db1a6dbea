#!/usr/bin/env python
"""Benchmark of the speculative-decoding verify path on one MI355X.

Default workload (the headline): fused verify, B=64 rows, k=4 drafts (5 target
positions per row), V=151,936, bf16 logits, T=0.8, top-p 0.95. One step =
one call of the verify path over one batch: fused to_probs on all 576 target
and draft rows, accept test, residual/bonus draw. Inputs (seeded synthetic
logits with a Zipf head, draft = target + N(0,1), draft ids drawn from q) are
resident in HBM; three input sets (525 MB, more than the 256 MB MALL) rotate so
no step reads another step's bytes from cache.

    python bench.py [--steps K] [--warmup W]
                    [--workload verify|greedy|kv|attn|ragged|probs|draft|round]

Prints one JSON line: verified tokens/s (sum over rows of n_acc + 1 per
step), the roofline of the fused verify step (algorithmic bytes = every logit
read once, over the step time measured with HIP events on the launch stream),
and the CPU baseline (the reference's op sequence in torch on the host's
cores, over the whole step of one input set).
"""
import argparse
import json
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "adaptive-specdec_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "verified tokens/sec at B=64,k=4,V=151936; % of HBM peak; speedup vs host CPU"
HBM_PEAK_GBS = 8000.0
STAT_CHAIN = 8
STEP_CHAIN = 16  # default of --chain


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def timed_graphs(graphs, steps, torch):
    """Replay graphs round-robin `steps` times between two events; ms per replay."""
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        graphs[i % len(graphs)].replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def timed_steps(chains, singles, steps, torch, chain):
    """Exactly `steps` verify steps: steps // chain replays of the chained
    graphs, then the remainder as single-step graphs, all between two events;
    ms per step."""
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps // chain):
        chains[i % len(chains)].replay()
    for i in range(steps % chain):
        singles[i % len(singles)].replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def capture(fn, torch):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def bench_verify(args, torch):
    import numpy as np
    from specdec.sampling import Verifier
    from specdec.workloads import verify_inputs

    B, k, V, T, tp = 64, 4, args.vocab, 0.8, 0.95
    dev = "cuda:0"
    log(f"generating {args.sets} input sets B={B} k={k} V={V}")
    sets = [verify_inputs(B, k, V, seed=1000 + i, device=dev, temperature=T, top_p=tp)
            for i in range(args.sets)]
    vers = [Verifier(B, k, V, torch.bfloat16, temperature=T, top_p=tp, device=dev)
            for _ in sets]
    calls = [(lambda v=v, s=s: v(s["target"], s["draft"], s["draft_ids"], s["u_accept"],
                                 s["u_final"])) for v, s in zip(vers, sets)]
    # the dominant kernel alone: row statistics of all 576 rows (no drafted tokens,
    # so no rank pass). Each graph holds STAT_CHAIN launches over rotating input
    # sets, so the per-launch time carries no graph-launch gap
    stat_calls = [(lambda v=v, s=s: v.stats(s["target"], s["draft"]))
                  for v, s in zip(vers, sets)]
    stat_chains = [(lambda i=i: [stat_calls[(i + j) % len(stat_calls)]()
                                 for j in range(STAT_CHAIN)])
                   for i in range(len(stat_calls))]
    # eager reference results, then warm up
    eager = []
    for c in calls:
        n, y, f = c()
        eager.append((n.clone(), y.clone(), f.clone()))
    for i in range(args.warmup):
        calls[i % len(calls)]()
        stat_calls[i % len(calls)]()
    torch.cuda.synchronize()
    tokens = [int((n + 1).sum().item()) for n, _, _ in eager]
    if args.no_graph:
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(args.steps):
            calls[i % len(calls)]()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        ms_single = ms
        stat_ms = None
    else:
        graphs = [capture(c, torch) for c in calls]
        sgraphs = [capture(c, torch) for c in stat_chains]
        for rep in range(3):                       # every replay must equal the eager result
            for g, v, (n, y, f) in zip(graphs, vers, eager):
                g.replay()
                torch.cuda.synchronize()
                ok = (torch.equal(v.n_acc, n) and torch.equal(v.y, y) and torch.equal(v.flags, f))
                if not ok:
                    raise RuntimeError("graph replay differs from the eager verify")
        # the timed graphs hold args.chain consecutive verify steps over the rotating
        # sets (as an engine's captured decode loop would), so the host's per-replay
        # launch cost is paid once per args.chain steps
        chains = [capture(lambda i=i: [calls[(i + j) % len(calls)]() for j in range(args.chain)],
                          torch) for i in range(len(calls))]
        ms = timed_steps(chains, graphs, args.steps, torch, args.chain)
        ms_single = timed_graphs(graphs, args.steps, torch)
        stat_ms = timed_graphs(sgraphs, max(args.steps // STAT_CHAIN, 10), torch) / STAT_CHAIN
    # eager timing too (host launch path), for the record
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(min(args.steps, 100)):
        calls[i % len(calls)]()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / min(args.steps, 100)

    value = (sum(tokens) / len(tokens)) / (ms / 1e3)
    rows = B * (2 * k + 1)
    alg_bytes = rows * V * 2                     # every bf16 logit read once
    out_bytes = B * (8 + 8 + 1)
    # the roofline is the whole verify step (one C-ABI call: one fused launch of
    # row statistics and draw, or the two kernels when SDX_VERIFY_FUSED=0),
    # timed over the timed region
    achieved = alg_bytes / (ms / 1e3) / 1e9
    fused = os.environ.get("SDX_VERIFY_FUSED", "1") != "0"
    roof = {"bound": "hbm",
            "kernel": ("verify_fused_bf16_kernel (row statistics + accept/draw, one launch)"
                       if fused else
                       "verify step: rowstream_bf16_kernel + draw16_kernel (two launches)"),
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            # the committed traffic figures were measured at V = 151936
            "traffic": traffic_per_launch() if fused and V == 151936 else None,
            "algorithmic_bytes": alg_bytes, "avg_launch_us": round(ms * 1e3, 2)}
    cpu = None if args.skip_cpu else cpu_baseline(sets[0], eager[0], args, T, tp, np, torch)
    result = {
        "metric": METRIC.replace("V=151936", f"V={V}"), "value": round(value, 1),
        "unit": "verified tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"fused verify B=64 k=4 V={V} bf16 T=0.8 top-p 0.95",
                   "batch": B, "k": k, "vocab": V, "logits": "bf16", "temperature": T,
                   "top_p": tp, "input_sets": len(sets), "hip_graph": not args.no_graph},
        "rows_per_s": round(rows / (ms / 1e3), 1),
        "step_bytes_algorithmic": alg_bytes + out_bytes,
        "step_hbm_frac": round((alg_bytes + out_bytes) / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
        "eager_ms_per_step": round(eager_ms, 4),
        "graph_per_step_ms_per_step": round(ms_single, 5),
        "row_stats_only_us": None if stat_ms is None else round(stat_ms * 1e3, 2),
        "mean_accepted": round(sum(tokens) / len(tokens) / B - 1, 4),
        # rows whose accept tests or final draw touched a partially kept top-p tie
        # group (SDX_FLAG_TIE_ORDER), over every input set
        "tie_order_rows": int(sum(int(((f & 32) != 0).sum().item()) for _, _, f in eager)),
        "rows_checked": B * len(eager),
        "roofline": roof, "cpu_baseline": cpu,
    }
    if cpu:
        result["speedup_vs_cpu"] = round(value / cpu["value"], 1)
    return result


def traffic_per_launch(name="traffic_verify.json"):
    """HBM bytes per step (or launch) of the roofline's kernels, from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE summary (scaled by the copy-kernel
    calibration), or None."""
    p = os.path.join(REPO, "profiles", name)
    try:
        with open(p) as f:
            return json.load(f).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def cpu_sockets():
    try:
        with open("/proc/cpuinfo") as f:
            ids = {line.split(":", 1)[1].strip() for line in f if line.startswith("physical id")}
        return max(len(ids), 1)
    except OSError:
        return None


def cpu_threads():
    """Threads for the CPU baseline: the cores this process may run on, capped by
    OMP_NUM_THREADS when the environment sets it (the host's share)."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return n


def cpu_baseline(s, eager, args, T, tp, np, torch):
    """The reference's verify path as torch CPU ops (`oracle/torch_path.py`:
    `to_probs` per position, then the accept block of `engine.py:281-312`) on the
    whole step of input set 0, on the host's cores: one warmup, then the median
    of `cpu_runs` runs. Its ids are compared with the GPU's."""
    from oracle import torch_path as TP
    nthr = cpu_threads()
    torch.set_num_threads(nthr)
    tl, dl = s["target"].cpu(), s["draft"].cpu()
    ids, ua, uf = s["draft_ids"].cpu(), s["u_accept"].cpu(), s["u_final"].cpu()
    B, k1, V = tl.shape
    log(f"cpu baseline: torch CPU path on the whole step, {nthr} threads")
    TP.rejection_sample(tl, dl, ids, ua, uf, T, tp, 0)
    times = []
    for _ in range(args.cpu_runs):
        t0 = time.perf_counter()
        n, y = TP.rejection_sample(tl, dl, ids, ua, uf, T, tp, 0)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    gn, gy = (t.cpu() for t in eager[:2])
    same = float(((n == gn) & (y == gy)).double().mean())
    toks = int((n + 1).sum())
    return {"value": round(toks / med, 1), "unit": "verified tokens/s", "cores": nthr,
            "kind": "port", "seconds_per_step": round(med, 4),
            "sample": f"the whole step of input set 0 (B={B}, k={k1 - 1}, {B * (2 * k1 - 1)} "
                      f"vocab rows of {V}), torch CPU ops, median of {len(times)} runs after "
                      f"one warmup",
            "cpu": cpu_model(), "sockets": cpu_sockets(),
            "threads_available": len(os.sched_getaffinity(0)),
            "rows_equal_gpu": round(same, 4)}


def bench_greedy(args, torch):
    from specdec.sampling import Verifier
    from specdec.workloads import greedy_inputs
    B, k, V = 256, 8, 151936
    dev = "cuda:0"
    sets = [greedy_inputs(B, k, V, seed=2000 + i, device=dev) for i in range(args.sets)]
    vers = [Verifier(B, k, V, torch.bfloat16, temperature=0.0, device=dev) for _ in sets]
    calls = [(lambda v=v, s=s: v(s["target"], None, s["draft_ids"], s["u_accept"],
                                 s["u_accept"][:, 0].contiguous())) for v, s in zip(vers, sets)]
    for i in range(args.warmup):
        calls[i % len(calls)]()
    torch.cuda.synchronize()
    tokens = []
    for c in calls:
        n, _, _ = c()
        tokens.append(int((n + 1).sum().item()))
    graphs = [capture(c, torch) for c in calls]
    ms = timed_graphs(graphs, args.steps, torch)
    alg = B * (k + 1) * V * 2
    value = sum(tokens[i % len(tokens)] for i in range(args.steps)) / (ms * args.steps / 1e3)
    ach = alg / (ms / 1e3) / 1e9
    return {"metric": "verified tokens/sec, greedy verify B=256,k=8,V=151936", "value": round(value, 1),
            "unit": "verified tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "greedy verify B=256 k=8 V=151936 bf16", "batch": B, "k": k,
                       "vocab": V},
            "roofline": {"bound": "hbm", "kernel": "argmax_kernel + greedy_accept_kernel",
                         "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                         "algorithmic_bytes": alg},
            "cpu_baseline": None}


def bench_kv(args, torch):
    from specdec.kvcache import PagedKVCache
    from specdec.workloads import kv_inputs
    L, B, q, H, D, bs = 64, 64, 5, 8, 128, 16
    dev = "cuda:0"
    inp = kv_inputs(L, B, q, H, D, bs, 512, 4096, seed=3, device=dev)
    c = PagedKVCache(L, B, inp["num_blocks"], bs, H, D, inp["max_blocks"], device=dev)
    c.block_table.copy_(inp["block_table"])
    c.lengths.copy_(inp["lengths"])
    drop = (q - inp["keep"]).contiguous()
    staged = inp["staged"]

    def step():
        c.append(staged)
        c.commit(q)
        c.rollback(drop)
        c.lengths.copy_(inp["lengths"])          # keep the workload stationary

    for _ in range(args.warmup):
        step()
    g = capture(step, torch)
    ms = timed_graphs([g], args.steps, torch)
    ga = capture(lambda: c.append(staged), torch)
    ms_append = timed_graphs([ga], args.steps, torch)
    alg = 2 * L * 2 * B * q * H * D * 2            # staged read + pool written
    ach = alg / (ms_append / 1e3) / 1e9
    return {"metric": "KV append+commit+rollback, 64 layers x B=64 x 5 pos, GB/s",
            "value": round(ach, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "paged KV append 64 layers, B=64, 5 positions, 8x128 bf16, "
                                   "block 16, seq 512-4096", "layers": L, "batch": B, "q": q},
            "roofline": {"bound": "hbm", "kernel": "kv_append_paged_kernel",
                         "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                         "algorithmic_bytes": alg, "avg_launch_us": round(ms_append * 1e3, 2)},
            "cpu_baseline": None}


def bench_probs(args, torch):
    """The standalone drop-ins the reference engine calls most (`engine.py:250,282`
    `to_probs`, `engine.py:301-302` `sample_from_probs`): 256 rows of V=151936
    bf16 logits (B=64 x k=4 draft positions), T=0.8, top-p 0.95 -> fp32
    probabilities, then one inverse-CDF draw per row from them. Each call is
    timed on its own, replayed from graphs over three rotating input sets.
    `--logits f32` feeds fp32 logits instead (the fp32 row kernel: each row
    read once, its probabilities written once)."""
    from specdec.sampling import sample_from_probs, to_probs
    from specdec.workloads import uniforms, zipf_logits
    rows, V, T, tp = 256, 151936, 0.8, 0.95
    f32 = args.logits == "f32"
    ldt = torch.float32 if f32 else torch.bfloat16
    isz = 4 if f32 else 2
    dev = "cuda:0"
    sets = []
    for i in range(3):
        g = torch.Generator(device=dev).manual_seed(2000 + i)
        sets.append((zipf_logits(rows, V, g, dev, dtype=ldt), uniforms((rows,), g, dev)))
    probs = [None] * 3

    def tp_step(i):  # captured: probs[i] is the graph's static output
        probs[i] = to_probs(sets[i][0], T, tp)

    def sp_step(i):
        sample_from_probs(probs[i], u=sets[i][1])

    for _ in range(max(1, args.warmup)):
        for i in range(3):
            tp_step(i)
            sp_step(i)
    gt = [capture(lambda i=i: tp_step(i), torch) for i in range(3)]
    gs = [capture(lambda i=i: sp_step(i), torch) for i in range(3)]
    ms_tp_call = timed_graphs(gt, args.steps, torch)
    ms_sp = timed_graphs(gs, args.steps, torch)
    # for reference: a plain fill of the same fp32 output (pure writes, torch's kernel)
    fills = [torch.empty(rows, V, dtype=torch.float32, device=dev) for _ in range(3)]
    gf = [capture(lambda f=f: f.fill_(0.5), torch) for f in fills]
    ms_fill = timed_graphs(gf, args.steps, torch)
    alg_tp = rows * V * (isz + 4)                   # logits in, fp32 probs out
    alg_sp = rows * V * 4                           # fp32 probs in
    ach_tp = alg_tp / (ms_tp_call / 1e3) / 1e9
    ach_sp = alg_sp / (ms_sp / 1e3) / 1e9
    lname = "f32" if f32 else "bf16"
    kname = "to_probs_f32_big_kernel" if f32 else "rowstream + materialize16"
    return {"metric": f"to_probs + sample_from_probs, 256 x 151936 {lname} logits, GB/s",
            "value": round((alg_tp + alg_sp) / ((ms_tp_call + ms_sp) / 1e3) / 1e9, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms_tp_call + ms_sp, 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": f"to_probs 256 x 151936 {lname} (T=0.8, top-p 0.95) -> fp32, "
                                   "then sample_from_probs on it", "rows": rows, "vocab": V},
            "to_probs_us": round(ms_tp_call * 1e3, 2),
            "sample_from_probs_us": round(ms_sp * 1e3, 2),
            "fill_output_us": round(ms_fill * 1e3, 2),
            "roofline": {"bound": "hbm",
                         "kernel": f"to_probs ({kname})",
                         "achieved": round(ach_tp, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach_tp / HBM_PEAK_GBS, 4), "traffic": None,
                         "algorithmic_bytes": alg_tp, "avg_launch_us": round(ms_tp_call * 1e3, 2)},
            "roofline_sample": {"bound": "hbm", "kernel": "sample_from_probs "
                                "(dense_mass + dense_pick)", "achieved": round(ach_sp, 1),
                                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(ach_sp / HBM_PEAK_GBS, 4), "traffic": None,
                                "algorithmic_bytes": alg_sp,
                                "avg_launch_us": round(ms_sp * 1e3, 2)},
            "cpu_baseline": None}


def bench_ragged(args, torch):
    """Config 5's sampler: B=128 rows with per-row k_b = best_k(alpha_b, 0.1),
    alpha_b ~ U(0.4, 0.9), V=151936 bf16 logits as in the fused verify, T=0.7,
    top-k 50, top-p 0.9; one call verifies all rows (packed [sum(k_b+1), V] and
    [sum k_b, V])."""
    from specdec.sampling import rejection_sample_ragged
    from specdec.workloads import ragged_verify_inputs
    B, V, T, tp, tk = 128, 151936, 0.7, 0.9, 50
    dev = "cuda:0"
    sets = [ragged_verify_inputs(B, V, seed=2000 + i, device=dev, temperature=T, top_p=tp, top_k=tk)
            for i in range(args.sets)]
    outs = [tuple(torch.empty(B, dtype=dt, device=dev) for dt in (torch.int64, torch.int64,
                                                                   torch.uint8)) for _ in sets]
    wss = [None] * len(sets)

    def call(i):
        s = sets[i]
        return rejection_sample_ragged(s["target"], s["draft"], s["draft_ids"], s["u_accept"],
                                       s["u_final"], s["cu_k"], k_max=8, temperature=T,
                                       top_p=tp, top_k=tk, workspace=wss[i], out=outs[i])
    from specdec import _lib
    for i, s in enumerate(sets):  # one workspace per input set, zero-filled once
        nt = s["target"].shape[0]
        wss[i] = _lib.workspace(_lib.lib().sdx_verify_ragged_workspace(B, nt, V, _lib.BF16), dev)
    eager = []
    for i in range(len(sets)):
        n, y, f = call(i)
        eager.append((n.clone(), y.clone(), f.clone()))
    for i in range(args.warmup):
        call(i % len(sets))
    torch.cuda.synchronize()
    graphs = [capture(lambda i=i: call(i), torch) for i in range(len(sets))]
    for rep in range(3):                       # every replay must equal the eager result
        for g, o, (n, y, f) in zip(graphs, outs, eager):
            g.replay()
            torch.cuda.synchronize()
            if not (torch.equal(o[0], n) and torch.equal(o[1], y) and torch.equal(o[2], f)):
                raise RuntimeError("graph replay differs from the eager verify")
    ms = timed_graphs(graphs, args.steps, torch)
    tokens = sum(int((n + 1).sum().item()) for n, _, _ in eager) / len(eager)
    rows = sum(int(s["target"].shape[0]) + int(s["draft"].shape[0]) for s in sets) / len(sets)
    alg = rows * V * 2
    ach = alg / (ms / 1e3) / 1e9
    mean_k = sum(sum(s["k"]) for s in sets) / (len(sets) * B)
    return {"metric": "verified tokens/sec, adaptive-k verify B=128 (per-row k), V=151936",
            "value": round(tokens / (ms / 1e3), 1), "unit": "verified tokens/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic",
            "config": {"workload": "adaptive-k fused verify B=128, k_b=best_k(U(0.4,0.9), c=0.1), "
                                   "V=151936 bf16, T=0.7 top-k 50 top-p 0.9",
                       "batch": B, "mean_k": round(mean_k, 3), "rows": rows,
                       "input_sets": len(sets), "hip_graph": True},
            "mean_accepted": round(tokens / B - 1, 4),
            "roofline": {"bound": "hbm", "kernel": "whole call (row statistics + draw)",
                         "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                         "algorithmic_bytes": int(alg), "avg_launch_us": round(ms * 1e3, 2)},
            "cpu_baseline": None}


def bench_attn(args, torch):
    """Adaptive-k verify attention, one layer: B=128 rows with k_b = best_k(alpha_b, 0.1),
    alpha_b ~ U(0.4, 0.9), contexts ~ U[1024, 8192], 32 query / 8 KV heads of 128,
    paged bf16 KV (block 16). HBM roofline: every visible key and value read once."""
    from specdec.attention import attention_workspace, verify_attention_paged
    from specdec.workloads import attn_inputs
    dev = "cuda:0"
    B = 128
    inp = attn_inputs(B, seed=5, device=dev)
    out = torch.empty_like(inp["q"])
    bs, mb = inp["k_pool"].shape[1], inp["block_table"].shape[1]
    ws = attention_workspace(B, inp["max_q"], inp["hq"], inp["hkv"], bs, mb, args.attn_chunk,
                             device=dev)
    call = lambda: verify_attention_paged(inp["q"], inp["cu_q"], inp["k_pool"], inp["v_pool"],  # noqa: E731
                                          inp["block_table"], inp["kv_len"], inp["max_q"],
                                          out=out, chunk_tokens=args.attn_chunk, workspace=ws)
    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()
    if args.no_graph:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            call()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
    else:
        g = capture(call, torch)
        ms = timed_graphs([g], args.steps, torch)
    kv_tokens = int(inp["kv_len"].sum().item())
    d, hkv, hq = inp["d"], inp["hkv"], inp["hq"]
    T = int(inp["cu_q"][-1].item())
    alg = kv_tokens * hkv * d * 2 * 2 + 2 * T * hq * d * 2   # K + V once, q in, out
    flops = 4 * d * sum(int(q) * hq * int(n) for q, n in
                        zip((inp["k"] + 1).tolist(), inp["kv_len"].tolist()))
    ach = alg / (ms / 1e3) / 1e9
    return {"metric": "verify attention (1 layer, paged KV), GB/s", "value": round(ach, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "adaptive-k verify attention B=128, k_b=best_k(U(0.4,0.9), c=0.1), "
                                   "ctx U[1024,8192], 32/8 heads x 128, paged bf16 block 16",
                       "batch": B, "query_rows": T, "kv_tokens": kv_tokens,
                       "chunk_tokens": args.attn_chunk,
                       "mean_k": round(float(inp["k"].float().mean()), 3)},
            "roofline": {"bound": "hbm",
                         "kernel": "whole call: verify_attn_plan + verify_attn_kernel + "
                                   "verify_attn_merge",
                         "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4),
                         "traffic": traffic_per_launch("traffic_attn.json"),
                         "algorithmic_bytes": alg, "avg_launch_us": round(ms * 1e3, 2),
                         "mfma_tflops": round(flops / (ms / 1e3) / 1e12, 2)},
            "cpu_baseline": None}


def bench_draft(args, torch):
    """One draft step of the device round (engine.py:246-258 with the early exit of
    controller.py:184-187): B=64 rows of V=151936 bf16 draft logits, T=0.8, top-p
    0.95; to_probs statistics, the inverse-CDF draw, q(x), conf *= q(x) and the
    early-exit flag, all on the device. HBM roofline: every logit read once."""
    from specdec import _lib
    from specdec.sampling import draft_step
    from specdec.workloads import uniforms, zipf_logits
    B, V, T, tp = 64, args.vocab, 0.8, 0.95
    dev = "cuda:0"
    g = torch.Generator(device=dev).manual_seed(3000)
    xs = [zipf_logits(B, V, g, dev) for _ in range(args.sets)]
    us = [uniforms((B,), g, dev) for _ in range(args.sets)]
    confs = [torch.ones(B, dtype=torch.float32, device=dev) for _ in range(args.sets)]
    outs = [(torch.empty(B, dtype=torch.int64, device=dev),
             torch.empty(B, dtype=torch.float32, device=dev),
             torch.zeros(1, dtype=torch.int32, device=dev)) for _ in range(args.sets)]
    L = _lib.lib()
    wss = [_lib.workspace(L.sdx_draft_step_workspace(B, V, _lib.BF16), dev)
           for _ in range(args.sets)]

    def call(i):
        return draft_step(xs[i], us[i], T, tp, 0, conf=confs[i], tau=0.3, step=2, min_k=1,
                          out=outs[i], workspace=wss[i])
    for i in range(args.warmup):
        call(i % args.sets)
    torch.cuda.synchronize()
    graphs = [capture(lambda i=i: call(i), torch) for i in range(args.sets)]
    ms = timed_graphs(graphs, args.steps, torch)
    alg = B * V * 2
    ach = alg / (ms / 1e3) / 1e9
    return {"metric": "draft steps/sec, B=64 V=151936 bf16 (to_probs + draw + q(x) + early exit)",
            "value": round(1e3 / ms, 1), "unit": "draft steps/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic",
            "config": {"workload": f"draft step B={B} V={V} bf16 T=0.8 top-p 0.95, conf + tau",
                       "batch": B, "input_sets": args.sets, "hip_graph": True},
            "roofline": {"bound": "hbm", "kernel": "whole draft step (all launches)",
                         "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                         "algorithmic_bytes": int(alg), "avg_launch_us": round(ms * 1e3, 2)},
            "cpu_baseline": None}


def bench_round(args, torch):
    """One speculative round of `SpecEngine` (engine.py:228-342) replayed from a HIP
    graph: k=4 draft forwards of the stand-in TinyLM draft, each followed by the
    fused draft step, the commit-only draft forward, one target forward over the
    5 positions, the fused verify and the round commit. B=64, V=151936 bf16 logits,
    T=0.8, top-p 0.95 (no checkpoints: seeded one-layer models whose lm_head dominates
    the model time). The round's verify takes the draft rows' statistics from its
    draft steps (`Verifier.drafted`). Reported beside the round: the sampling path
    alone, the k draft steps, the verify as the round runs it and the verify that
    streams the draft rows too, on the round's own logits, each replayed from its
    own graph."""
    from specdec.engine import SpecEngine
    from specdec.tinylm import TinyLM
    B, k, V, T, tp = 64, 4, args.vocab, 0.8, 0.95
    dev = "cuda:0"
    tgt = TinyLM(V, hq=2, hkv=1, seed=1, device=dev, scale=4.0)
    drf = TinyLM(V, hq=2, hkv=1, seed=2, device=dev, base=tgt, noise=0.6)
    P = 16
    rounds_max = args.steps + args.warmup + 8
    max_new = rounds_max * (k + 1) + 2
    eng = SpecEngine(tgt, drf, B, k, temperature=T, top_p=tp, max_new=max_new, prompt_len=P,
                     device=dev, observe_cost=False)
    gen = torch.Generator(device="cpu").manual_seed(7)
    prompt = torch.randint(0, V, (B, P), generator=gen).to(dev)
    g = torch.Generator(device=dev).manual_seed(11)
    eng.start(prompt, u_first=torch.rand(B, generator=g, device=dev))
    torch.rand(eng.u_draft.shape, generator=g, device=dev, out=eng.u_draft)
    torch.rand(eng.u_acc.shape, generator=g, device=dev, out=eng.u_acc)
    torch.rand(eng.u_fin.shape, generator=g, device=dev, out=eng.u_fin)
    tokens = []
    for _ in range(max(args.warmup, 2)):           # eager rounds (the capture needs one)
        n_acc, _ = eng.round(k)
        tokens.append(int((n_acc + 1).sum().item()))
    graph = eng.capture(k)
    torch.cuda.synchronize()
    ms = timed_graphs([graph], args.steps, torch)
    torch.cuda.synchronize()
    # the sampling path alone on the last round's logits: k draft steps, then the verify
    from specdec.sampling import draft_step
    dlog = eng.dlog.clone()
    tlog = eng.last_target_logits.contiguous().clone()
    xs, ua, uf = eng.xs.clone(), eng.u_acc.clone(), eng.u_fin.clone()
    ud = eng.u_draft.clone()
    conf = torch.ones(B, dtype=torch.float32, device=dev)
    douts = [eng.step_out[i] for i in range(k)]
    dws = eng.draft_ws

    def steps():
        for i in range(k):
            draft_step(dlog[:, i], ud[i], T, tp, 0, out=douts[i], workspace=dws[i])
    ver = eng._verifier(k)

    def verify():
        ver(tlog, dlog, xs, ua, uf)

    def verify_drafted():
        ver.drafted(tlog, dlog, xs, ua, uf, dws)
    for _ in range(3):
        steps()
        verify()
        verify_drafted()
    gs, gv, gd = capture(steps, torch), capture(verify, torch), capture(verify_drafted, torch)
    ms_steps = timed_graphs([gs], args.steps, torch)
    ms_verify = timed_graphs([gv], args.steps, torch)
    ms_drafted = timed_graphs([gd], args.steps, torch)
    tok = sum(tokens) / len(tokens)
    return {"metric": "speculative rounds/sec, TinyLM pair B=64 k=4 V=151936 (graph replay)",
            "value": round(1e3 / ms, 2), "unit": "rounds/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded one-layer models, no checkpoint)",
            "config": {"workload": f"SpecEngine round B={B} k={k} V={V} bf16 T=0.8 top-p 0.95",
                       "batch": B, "k": k, "prompt_len": P, "hip_graph": True},
            "tokens_per_round": round(tok, 2),
            "tokens_per_s": round(tok / (ms / 1e3), 1),
            "draft_steps_ms": round(ms_steps, 5), "verify_ms": round(ms_verify, 5),
            "verify_drafted_ms": round(ms_drafted, 5),
            "sampling_share": round((ms_steps + ms_drafted) / ms, 4),
            "roofline": None, "cpu_baseline": None}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="verify",
                    choices=["verify", "greedy", "kv", "attn", "ragged", "probs", "draft",
                             "round"])
    ap.add_argument("--sets", type=int, default=3)
    ap.add_argument("--vocab", type=int, default=151936,
                    help="verify workload: vocabulary of the bf16 rows (151936: the headline)")
    ap.add_argument("--attn-chunk", type=int, default=0,
                    help="attn workload: keys per chunk (0: the library default)")
    ap.add_argument("--logits", default="bf16", choices=["bf16", "f32"],
                    help="probs workload: dtype of the logits")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--chain", type=int, default=STEP_CHAIN,
                    help="verify steps per timed graph replay (the headline workload)")
    ap.add_argument("--cpu-runs", type=int, default=5)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 256 MiB device copy (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the verify path is row-parallel "
              "and shards by batch rows without communication); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no ROCm device visible", file=sys.stderr)
        sys.exit(1)
    fn = {"verify": bench_verify, "greedy": bench_greedy, "kv": bench_kv,
          "attn": bench_attn, "ragged": bench_ragged, "probs": bench_probs,
          "draft": bench_draft, "round": bench_round}[args.workload]
    result = fn(args, torch)
    if args.calibrate_copy:
        # a device-to-device copy of known size: its FETCH_SIZE / WRITE_SIZE per
        # dispatch scale the same counters of the verify kernels to bytes
        n = 256 << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: 5 x {n} bytes")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()

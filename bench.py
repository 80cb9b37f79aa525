"""Benchmark of the DSA decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg2]

A step is one call of ``dsa_amd.kernel`` (the drop-in for the reference's
``kernel()``, solution/triton/kernel.py:138) on the BASELINE decode workload:
T=64 tokens, H=16, top-k=2048, ckv512+kpe64 bf16, 131072 slots in pages of 64
(config 2).  Inputs are synthetic, seeded, and resident in HBM before timing.
Steps are captured 20 at a time in a HIP graph and the graph is replayed, so
the figure is the GPU time of back-to-back calls rather than Python/ctypes
launch overhead (the eager per-call time is reported alongside).  Timing uses
HIP events on the stream the kernels run on: W untimed warm-up steps, then K
timed steps between synchronisations.  The dominant kernel is the gather
attention: at H=16 a call is that one launch (the split merge runs inside
it), so the graph time per call is its duration; for head counts whose calls
add a separate merge launch it is timed on its own through
dsa_attn_fwd_partial.  That duration gives the roofline figure.

Prints one JSON line (metric, value in us/call, roofline of the dominant
kernel, and a CPU baseline: the CPU oracle timed on this host).  Repeated
calls on one 151 MB cache find it in the 256 MB Infinity Cache; for cfg2 the
line also carries ``config.cold_cache``: the same calls rotating through 3
copies of the cache (453 MB), so the gathers come from HBM.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "flashinfer-repo_amd")]

METRIC = "µs/call + HBM GB/s & MFMA %, DSA decode H=16 topk=2048 T=64"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
INT8_PEAK_TOPS = 5000.0      # dense int8 MFMA (= the fp8 dense peak)
GRAPH_CALLS = 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="cfg2", choices=["cfg1", "cfg2", "cfg3", "cfg4", "cfg5"],
                    help="cfg1-cfg4: sparse attention; cfg5: lightning indexer + top-k "
                         "feeding the cfg2 attention")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="budget of the CPU-oracle baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cold-copies", type=int, default=-1, metavar="N",
                    help="also time calls that rotate through N copies of the KV cache, so no "
                         "call finds its rows in the 256 MB Infinity Cache (default: 3 for cfg2, "
                         "whose cache is 151 MB; 0 = off)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run 5 plain device copies of BYTES bytes (the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    return ap.parse_args()


def copy_calibration(nbytes: int) -> None:
    import torch
    src = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "copies": 5}), flush=True)


def load_traffic(config: str):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    ent = t.get(config)
    return None if ent is None else ent.get("hbm_bytes_per_launch")


def cpu_baseline(d, budget_s: float):
    """Times the CPU oracle (the restatement of the reference's run()) on the
    same workload, whole calls, until the budget is spent."""
    import numpy as np
    import torch

    import oracle

    def bits(t):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)

    args = (bits(d["q_nope"]), bits(d["q_pe"]), bits(d["ckv_cache"]), bits(d["kpe_cache"]),
            d["sparse_indices"].numpy(), d["sm_scale"])
    threads = min(16, os.cpu_count() or 1)
    oracle.attention(*args, nthreads=threads)  # warm-up (page-in, thread pool)
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.attention(*args, nthreads=threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 1000:
            break
    T = d["q_nope"].shape[0]
    return {"value": el / n * 1e6, "unit": "µs/call", "cores": threads, "kind": "port",
            "sample": f"{n} full calls of the {T}-token workload (fp64 CPU oracle, OpenMP "
                      f"{threads} threads, {el:.1f} s)"}


def graph_of(fn, n):
    """Capture n back-to-back calls of fn in one HIP graph (after an eager
    warm-up on the capture-side stream, as torch's graph API expects)."""
    import torch
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for _ in range(n):
            fn()
    torch.cuda.synchronize()
    return graph


def time_graph(graph, n_per, steps, warmup):
    """ms per call: warm-up replays, then HIP events around the replays (on
    the current stream, which the kernels run on)."""
    import torch
    reps = max(1, -(-steps // n_per))
    for _ in range(max(1, -(-warmup // n_per))):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (reps * n_per), reps * n_per


def time_eager(fn, steps):
    import torch
    fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def cpu_indexer_baseline(d, budget_s: float):
    """Times the CPU oracle's exact indexer score + top-k on a bounded sample
    of the cfg5 rows (whole rows of all positions)."""
    import numpy as np

    import oracle
    threads = min(16, os.cpu_count() or 1)
    T = d["q_idx"].shape[0]
    lim = d["causal_limit"].numpy().astype(np.int64)
    qa, ka = d["q_idx"].numpy(), d["k_idx"].numpy()
    sc, w = d["k_scale"].numpy(), d["weights"].numpy()
    rows = 4
    oracle.indexer_scores(qa[:1], ka, sc, w[:1], lim[:1], threads)  # warm-up
    n, t0 = 0, time.perf_counter()
    while True:
        i = (n * rows) % T
        s = oracle.indexer_scores(qa[i:i + rows], ka, sc, w[i:i + rows], lim[i:i + rows], threads)
        oracle.topk(s, lim[i:i + rows], int(d["topk"]))
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n * rows >= 10 * T:
            break
    per_call = el / (n * rows) * T
    return {"value": per_call * 1e6, "unit": "µs/call", "cores": threads, "kind": "port",
            "sample": f"{n * rows} of {T} token rows (exact score over all positions + top-k, "
                      f"OpenMP {threads} threads, {el:.1f} s), scaled to the {T}-row call"}


def bench_indexer(a):
    """cfg5: the lightning indexer + top-k (block-table slots) and the whole
    indexer -> attention pipeline."""
    import torch

    from dsa_amd import kernel, workloads
    from dsa_amd.indexer_kernel import run_indexer_and_topk

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    d = workloads.cfg5()
    g = workloads.to_device(d, dev)
    T, Hi, D = d["q_idx"].shape
    S = d["k_idx"].shape[0]
    K = int(d["topk"])
    ia = (g["q_idx"], g["k_idx"], g["k_scale"], g["weights"], g["causal_limit"])
    slots = run_indexer_and_topk(*ia, K, block_table=g["block_table"], page_size=64)
    attn = (g["q_nope"], g["q_pe"], g["ckv_cache"], g["kpe_cache"])

    def indexer():
        run_indexer_and_topk(*ia, K, block_table=g["block_table"], page_size=64)

    def scores_only():
        run_indexer_and_topk(*ia, 0, return_scores=True)

    def pipeline():
        sl = run_indexer_and_topk(*ia, K, block_table=g["block_table"], page_size=64)
        kernel(*attn, sl, d["sm_scale"])

    per_graph = min(GRAPH_CALLS, a.steps)
    ms_idx, timed_steps = time_graph(graph_of(indexer, per_graph), per_graph, a.steps, a.warmup)
    ms_score, _ = time_graph(graph_of(scores_only, per_graph), per_graph, a.steps, a.warmup)
    ms_pipe, _ = time_graph(graph_of(pipeline, per_graph), per_graph, a.steps, a.warmup)
    eager_ms = time_eager(pipeline, a.steps)

    ops = 2 * T * Hi * S * D                          # algorithmic dot-product ops
    tops = ops / (ms_score * 1e-3) / 1e12
    line = {
        "metric": "µs/call, lightning indexer + top-k -> DSA attention (cfg5)",
        "value": round(ms_pipe * 1e3, 3),
        "unit": "µs/call",
        "n_gpus": 1,
        "steps": timed_steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_pipe, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3 scores (exact), bf16 attention",
        "data": "synthetic (seeded; q_idx,k_idx ~N(0,1) as e4m3, scale~U(0.5,2), w~N(0,1/8))",
        "config": {"workload": f"cfg5: indexer T={T} heads={Hi} dim={D} positions={S} "
                               f"top-{K} -> block-table slots -> cfg2 attention H=16",
                   "timing": f"HIP graphs of {per_graph} back-to-back calls, replayed",
                   "indexer_topk_us": round(ms_idx * 1e3, 3),
                   "score_kernels_us": round(ms_score * 1e3, 3),
                   "topk_kernel_us": round((ms_idx - ms_score) * 1e3, 3),
                   "attention_us": round((ms_pipe - ms_idx) * 1e3, 3),
                   "eager_pipeline_us": round(eager_ms * 1e3, 3)},
        "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4),
                     "traffic": None, "algorithmic_ops": ops,
                     "kernel": "dsa_idx_prep_q_kernel + dsa_idx_score_kernel (timed via "
                               "dsa_indexer_topk with topk=0)"},
    }
    del slots
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = cpu_indexer_baseline(d, a.cpu_seconds)
    print(json.dumps(line), flush=True)


def main():
    a = parse()
    if a.copy_calibration:
        copy_calibration(a.copy_calibration)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for {max(a.gpus, world)}); "
              "the DSA path shards by tokens/heads with no exchange and is benchmarked at N=1.",
              file=sys.stderr)
        sys.exit(2)

    if a.config == "cfg5":
        bench_indexer(a)
        return

    import torch

    from dsa_amd import _lib, kernel, kernel_partial, num_splits, workloads

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    d = workloads.CONFIGS[a.config]()
    g = workloads.to_device(d, dev)
    T, H, _ = d["q_nope"].shape
    K = d["sparse_indices"].shape[1]
    args = (g["q_nope"], g["q_pe"], g["ckv_cache"], g["kpe_cache"], g["sparse_indices"],
            d["sm_scale"])
    alg_bytes = workloads.attention_bytes(d["sparse_indices"])
    alg_flops = workloads.attention_flops(d["sparse_indices"], H)

    per_graph = min(GRAPH_CALLS, a.steps)
    step_graph = graph_of(lambda: kernel(*args), per_graph)
    ms_per_step, timed_steps = time_graph(step_graph, per_graph, a.steps, a.warmup)

    # The dominant kernel.  When a kernel() call is one launch (one chunk per
    # token, or the split merge done inside the attention kernel) that launch
    # is the whole call; otherwise the gather-attention launch is timed alone
    # (dsa_attn_fwd_partial) and the merge kernel accounts for the rest.
    splits = num_splits(T, H, K)
    one_launch = splits == 1 or _lib.load().dsa_attn_counter_bytes(T, H) > 0
    if one_launch:
        ms_partial = ms_per_step
        kdesc = ("dsa_attn_ring_kernel (gather attention"
                 + (" with the split merge inside" if splits > 1 else "")
                 + "; the only launch of a kernel() call)")
    else:
        part_graph = graph_of(lambda: kernel_partial(*args, num_splits=0), per_graph)
        ms_partial, _ = time_graph(part_graph, per_graph, a.steps, a.warmup)
        kdesc = "dsa_attn_ring_kernel (per-chunk gather attention; timed alone via dsa_attn_fwd_partial)"

    # eager (Python shim + ctypes + launches) for reference
    eager_ms = time_eager(lambda: kernel(*args), a.steps)

    # Cold-cache variant: consecutive calls read different copies of the cache,
    # together larger than the Infinity Cache, so the gathers come from HBM.
    n_cold = a.cold_copies if a.cold_copies >= 0 else (3 if a.config == "cfg2" else 0)
    cold = None
    if n_cold > 0:
        copies = [(g["ckv_cache"].clone(), g["kpe_cache"].clone()) for _ in range(n_cold)]
        state = {"i": 0}

        def cold_call():
            c, k = copies[state["i"] % n_cold]
            state["i"] += 1
            kernel(g["q_nope"], g["q_pe"], c, k, g["sparse_indices"], d["sm_scale"])

        per = n_cold * max(1, per_graph // n_cold)
        ms_cold, _ = time_graph(graph_of(cold_call, per), per, a.steps, a.warmup)
        cold = {"copies": n_cold,
                "cache_bytes_per_copy": (g["ckv_cache"].numel() + g["kpe_cache"].numel()) * 2,
                "us_per_call": round(ms_cold * 1e3, 3),
                "gathered_GBps": round(alg_bytes / (ms_cold * 1e-3) / 1e9, 1)}
        del copies

    us = ms_per_step * 1e3
    gbs = alg_bytes / (ms_partial * 1e-3) / 1e9          # dominant kernel
    tflops = alg_flops / (ms_partial * 1e-3) / 1e12
    traffic = load_traffic(a.config)
    line = {
        "metric": METRIC if a.config == "cfg2" else
                  f"µs/call + HBM GB/s & MFMA %, DSA sparse attention H={H} topk={K} T={T} ({a.config})",
        "value": round(us, 3),
        "unit": "µs/call",
        "n_gpus": 1,
        "steps": timed_steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded; q~N(0,1), cache~N(0,0.5), distinct slots per token)",
        "config": {"workload": f"{a.config}: DSA sparse attention T={T} H={H} topk={K} "
                               f"ckv512+kpe64 bf16, {d['ckv_cache'].numel() // 512} slots, "
                               f"page_size={d['ckv_cache'].shape[1]}",
                   "tokens": T, "heads": H, "topk": K, "splits": splits,
                   "timing": f"HIP graphs of {per_graph} back-to-back kernel() calls, replayed",
                   "eager_us_per_call": round(eager_ms * 1e3, 3),
                   "cold_cache": cold,
                   "launches_per_call": 1 if one_launch else 2,
                   "dominant_kernel_us": round(ms_partial * 1e3, 3),
                   "merge_and_gaps_us": round((ms_per_step - ms_partial) * 1e3, 3)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "algorithmic_bytes": alg_bytes,
                     "kernel": kdesc},
        "mfma": {"achieved_tflops": round(tflops, 2), "peak_tflops": BF16_PEAK_TFLOPS,
                 "frac": round(tflops / BF16_PEAK_TFLOPS, 5), "algorithmic_flops": alg_flops},
    }
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(d, a.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

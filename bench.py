"""Benchmark of the DSA sparse-attention hot path on one MI355X.

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
attention: where a call is that one launch (the split merge inside it, or no
split) the graph time per call is its duration; otherwise it is timed on its
own through dsa_attn_fwd_partial.  That duration gives the roofline figure.

The default run prints one JSON line for config 2 (metric, value in us/call,
roofline of the dominant kernel, the CPU baseline) and carries the other
workloads under ``workloads``: config 1, prefill config 3 (roofline
``mfma``), config 4 (H=128), config 5 (indexer + top-k -> attention) and
``t1``, the shape of the reference's only published timing (T=1, 8462 pages),
next to its RTX 6000 Ada figures.  ``--config X`` prints the line of one
workload only (for profiler runs).

Repeated calls on one 151 MB cache find it in the 256 MB Infinity Cache; the
config 2 line also carries ``config.cold_cache``: the same calls rotating
through 3 copies of the cache (453 MB), so the gathers come from HBM.

``roofline.traffic`` is the HBM bytes per launch that rocprofv3 counters
measured (profiles/traffic.json), used only when that record was made from
the kernel sources of this tree (its csrc hash matches); otherwise null.

The CPU baseline is the torch fp32 restatement of the reference's run()
(oracle/torch_ref.py: whole-cache fp32 conversion, then a per-token loop) on
the host's cores, 1 warm-up and 3 timed calls, median -- a reported
baseline, not a target.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "flashinfer-repo_amd")]

METRIC = "µs/call + HBM GB/s & MFMA %, DSA decode H=16 topk=2048 T=64"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
INT8_PEAK_TOPS = 5000.0      # dense int8 MFMA (= the fp8 dense peak)
GRAPH_CALLS = 20
WARMUP_S = 0.05              # minimum untimed warm-up (seconds of graph replays) per timing
EXTRA_STEPS = 100            # timed calls per extra workload of the default run
ATTN_CONFIGS = ("cfg1", "cfg2", "cfg3", "cfg4", "t1")
# Workloads whose cache fits the 256 MB Infinity Cache also get a cold-cache
# figure: calls rotating through this many copies of the cache.
COLD_COPIES = {"cfg2": 3, "cfg4": 4}

# The reference's published T=1 figures (RTX 6000 Ada, docs/PROFILING.md:47-48,
# docs/SPLITK_OPTIMIZATION.md:140-148,159-163) -- context for the t1 workload.
T1_REFERENCE = {"hardware": "NVIDIA RTX 6000 Ada (reference docs)",
                "dsa_fwd_kernel_us": 92.4, "kernel_wall_us": 97.0,
                "best_splitk_wall_us": 68.3, "best_splitk_forward_kernel_us": 4.29,
                "sources": "docs/PROFILING.md:47-48, docs/SPLITK_OPTIMIZATION.md:140-163"}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default=None, choices=list(ATTN_CONFIGS) + ["cfg5"],
                    help="only this workload (default: cfg2 with every other workload "
                         "carried in the line)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cold-copies", type=int, default=-1, metavar="N",
                    help="also time calls rotating through N copies of the KV cache "
                         "(default: cfg2 3 copies, 453 MB, and cfg4 4 copies, 302 MB, beyond "
                         "the 256 MB Infinity Cache; 0 = off)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run 5 plain device copies of BYTES bytes (the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    ap.add_argument("--record-profiles", default=None, metavar="OUT_DIR",
                    help="run rocprofv3 over --config X of every workload (kernel trace, then "
                         "one counter pass each: FETCH_SIZE, WRITE_SIZE, MFMA busy, L2 hits) "
                         "and the copy calibration, raw output under OUT_DIR; write "
                         "profiles/traffic.json (with the kernel sources' hash) and one "
                         "summary per workload under profiles/ (this process never touches "
                         "the GPU)")
    ap.add_argument("--profile-configs", default=",".join(ATTN_CONFIGS + ("cfg5",)),
                    help="workloads --record-profiles covers (comma-separated)")
    ap.add_argument("--profiles-dir", default=os.path.join(ROOT, "profiles"),
                    help="where --record-profiles writes traffic.json and the summaries")
    return ap.parse_args()


def copy_calibration(nbytes: int) -> None:
    import torch
    src = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "copies": 5}), flush=True)


def csrc_hash() -> str:
    """sha256 over the kernel and ABI sources (the code a traffic record measured)."""
    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "flashinfer-repo_amd", "csrc")
    files = sorted(os.path.join(csrc, f) for f in os.listdir(csrc)
                   if f.endswith((".hip", ".cpp", ".h")))
    for p in files + [os.path.join(ROOT, "include", "dsa_abi.h")]:
        h.update(os.path.basename(p).encode())
        with open(p, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def load_record(config: str):
    """The committed rocprofv3 --pmc record of this workload's dominant kernel
    (profiles/traffic.json), or None when none exists or it was made from
    other kernel sources."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    ent = t.get(config)
    if not ent or ent.get("csrc_sha256") != csrc_hash():
        return None
    return ent


def load_traffic(config: str):
    """HBM bytes per launch of the dominant kernel (FETCH_SIZE + WRITE_SIZE,
    copy-calibrated) from the record, or None."""
    ent = load_record(config)
    return ent.get("hbm_bytes_per_launch") if ent else None


def load_counters(config: str):
    """Counter-derived figures of the record: MFMA busy fraction
    (SQ_VALU_MFMA_BUSY_CYCLES over 4 x SQ_BUSY_CU_CYCLES), L2 hit fraction
    (TCC_HIT / (TCC_HIT + TCC_MISS)), fetched and written bytes; or None."""
    ent = load_record(config)
    if not ent:
        return None
    return {k: ent.get(k) for k in ("mfma_busy_frac", "l2_hit_frac", "lds_busy_frac",
                                    "lds_bank_conflict_frac", "fetch_bytes_per_launch",
                                    "write_bytes_per_launch", "source")}


def host_cpu():
    """(model name, logical CPUs) of this host."""
    model = None
    try:
        out = subprocess.run(["lscpu"], stdout=subprocess.PIPE, stderr=subprocess.DEVNULL,
                             text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return model, os.cpu_count()


def cpu_baseline(d, budget_s: float = 20.0):
    """The torch fp32 restatement of run() (oracle/torch_ref.py) on the host:
    1 warm-up and up to 3 timed whole calls, median; fewer timed calls when
    the calls so far have used up ``budget_s`` (the long prefill shapes)."""
    import torch

    from oracle.torch_ref import run_fp32
    threads = torch.get_num_threads()   # the box's CPU share (OMP_NUM_THREADS) of the host
    args = (d["q_nope"], d["q_pe"], d["ckv_cache"], d["kpe_cache"], d["sparse_indices"],
            d["sm_scale"])
    t0 = time.perf_counter()
    run_fp32(*args)
    spent = time.perf_counter() - t0
    times = []
    while len(times) < 3 and (not times or spent + times[-1] <= budget_s):
        t0 = time.perf_counter()
        run_fp32(*args)
        times.append(time.perf_counter() - t0)
        spent += times[-1]
    times.sort()
    model, ncpu = host_cpu()
    T = d["q_nope"].shape[0]
    return {"value": round(times[len(times) // 2] * 1e6, 1), "unit": "µs/call", "cores": threads,
            "kind": "port",
            "sample": f"whole {T}-token calls of the torch fp32 restatement of run() "
                      f"(indexer_kernel.py:436-497: whole-cache fp32 conversion, per-token "
                      f"loop), median of {len(times)} after 1 warm-up: "
                      f"{', '.join(f'{x:.3f}' for x in times)} s",
            "host": {"lscpu_model": model, "logical_cpus": ncpu, "torch_threads": threads}}


def cpu_indexer_baseline(d, budget_s: float = 10.0):
    """The exact-score CPU oracle + top-k on a bounded sample of cfg5's rows
    (whole rows over all positions), scaled to the 64-row call."""
    import numpy as np
    import torch

    import oracle
    threads = torch.get_num_threads()
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
        if el >= budget_s or n * rows >= 2 * T:
            break
    return {"value": round(el / (n * rows) * T * 1e6, 1), "unit": "µs/call", "cores": threads,
            "kind": "port",
            "sample": f"{n * rows} token rows, cycling over the call's {T} (exact score over all "
                      f"positions + top-k, {threads} threads, {el:.1f} s), scaled to the {T}-row call"}


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


def time_graph(fn, steps, warmup, per=GRAPH_CALLS):
    """ms per call over exactly `steps` calls of fn: HIP graphs of `per`
    back-to-back calls (and one graph of the remainder when `per` does not
    divide `steps`), warm-up replays, then HIP events around the replays (on
    the current stream, which the kernels run on).  Returns (ms, steps)."""
    import torch
    per = max(1, min(per, steps))
    full, rest = divmod(steps, per)
    g_full = graph_of(fn, per)
    g_rest = graph_of(fn, rest) if rest else None
    # untimed warm-up: at least `warmup` calls and about WARMUP_S of replays,
    # so the first workload after a switch is not timed while the clocks and
    # the address translation of its buffers are still settling
    reps, t0 = 0, time.perf_counter()
    while reps < max(1, -(-warmup // per)) or time.perf_counter() - t0 < WARMUP_S:
        g_full.replay()
        reps += 1
        if reps % 8 == 0 or reps >= max(1, -(-warmup // per)):
            torch.cuda.synchronize()
    if g_rest is not None:
        g_rest.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(full):
        g_full.replay()
    if g_rest is not None:
        g_rest.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps, steps


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


def measure_attention(name, d, steps, warmup, cold_copies=0):
    """Times kernel() on workload d; returns the fields of its line."""
    import torch

    from dsa_amd import (_lib, kernel, kernel_out, kernel_partial, new_split_counters, new_workspace,
                         num_splits, workloads)
    g = workloads.to_device(d, "cuda:0")
    T, H, _ = d["q_nope"].shape
    K = d["sparse_indices"].shape[1]
    args = (g["q_nope"], g["q_pe"], g["ckv_cache"], g["kpe_cache"], g["sparse_indices"],
            d["sm_scale"])
    alg_bytes = workloads.attention_bytes(d["sparse_indices"])
    alg_flops = workloads.attention_flops(d["sparse_indices"], H)
    per_graph = min(GRAPH_CALLS, steps)
    ms, timed = time_graph(lambda: kernel(*args), steps, warmup)

    # The dominant kernel: a call of one launch (one chunk per token, or the
    # split merge inside the attention kernel) is that launch; otherwise the
    # gather-attention launch is timed alone and the merge kernel is the rest.
    splits = num_splits(T, H, K)
    groups = H // 16
    # kernel() brings split counters; the library merges inside the attention
    # kernel where they exist (odd group counts) and the call has at most 4
    # splits
    one_launch = splits == 1 or _lib.load().dsa_attn_call_counter_bytes(T, H, K, 0) > 0
    # four independent waves per head group for odd group counts and for even
    # ones whose T x splits x groups workgroups fit the 256 CUs; else the
    # shared-ring layout
    kname = ("dsa_attn_wave_kernel" if groups % 2 or T * splits * groups <= 256
             else "dsa_attn_ring_kernel")
    if one_launch:
        ms_dom = ms
        kdesc = (f"{kname} (gather attention"
                 + (" with the split merge inside" if splits > 1 else "")
                 + "; the only launch of a kernel() call)")
    else:
        ms_dom, _ = time_graph(lambda: kernel_partial(*args, num_splits=0), steps, warmup)
        kdesc = f"{kname} (per-chunk gather attention; timed alone via dsa_attn_fwd_partial)"
    eager_ms = time_eager(lambda: kernel(*args), steps)
    # the same without allocation: the destination-passing entry with
    # preallocated output, lse, workspace and split counters
    out = torch.empty_like(g["q_nope"])
    lse = torch.empty(g["q_nope"].shape[:2], dtype=torch.float32, device=g["q_nope"].device)
    ws = new_workspace(g["q_nope"], K)
    cnt = new_split_counters(g["q_nope"])
    eager_dps_ms = time_eager(lambda: kernel_out(*args, out, lse, workspace=ws, split_counters=cnt),
                              steps)
    del out, lse, ws, cnt

    cold = None
    if cold_copies > 0:
        copies = [(g["ckv_cache"].clone(), g["kpe_cache"].clone()) for _ in range(cold_copies)]
        state = {"i": 0}

        def cold_call():
            c, k = copies[state["i"] % cold_copies]
            state["i"] += 1
            kernel(g["q_nope"], g["q_pe"], c, k, g["sparse_indices"], d["sm_scale"])

        per = cold_copies * max(1, per_graph // cold_copies)
        ms_cold, _ = time_graph(cold_call, steps, warmup, per)
        cold = {"copies": cold_copies,
                "cache_bytes_per_copy": (g["ckv_cache"].numel() + g["kpe_cache"].numel()) * 2,
                "us_per_call": round(ms_cold * 1e3, 3),
                "gathered_GBps": round(alg_bytes / (ms_cold * 1e-3) / 1e9, 1),
                "frac_of_hbm_peak": round(alg_bytes / (ms_cold * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "TFLOPs": round(alg_flops / (ms_cold * 1e-3) / 1e12, 2),
                "frac_of_bf16_peak": round(alg_flops / (ms_cold * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                                           5)}
        del copies

    gbs = alg_bytes / (ms_dom * 1e-3) / 1e9
    tflops = alg_flops / (ms_dom * 1e-3) / 1e12
    hbm = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": load_traffic(name),
           "algorithmic_bytes": alg_bytes, "kernel": kdesc, "counters": load_counters(name)}
    mfma = {"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 5),
            "traffic": hbm["traffic"], "algorithmic_flops": alg_flops, "kernel": kdesc,
            "counters": hbm["counters"]}
    # Config 3 is the MFMA-bound shape by the target's definition (its gathers
    # hit a 40 MB causal window the caches hold), and config 4 is the dense
    # contraction with 128 heads on the MFMA M dimension (its counters show the
    # MFMA pipe, not HBM, as the busy unit); the others are priced against
    # HBM, with the MFMA fraction beside it.
    roofline, other = (mfma, hbm) if name in ("cfg3", "cfg4") else (hbm, mfma)
    cache_slots = d["ckv_cache"].numel() // 512
    ps = d["ckv_cache"].shape[1] if d["ckv_cache"].dim() == 3 else 1
    return {
        "us": ms * 1e3, "ms": ms, "timed": timed,
        "config": {"workload": f"{name}: DSA sparse attention T={T} H={H} topk={K} "
                               f"ckv512+kpe64 bf16, {cache_slots} slots, page_size={ps}",
                   "tokens": T, "heads": H, "topk": K, "splits": splits,
                   "timing": f"HIP graphs of {per_graph} back-to-back kernel() calls, replayed "
                             f"(plus one graph of the remainder): {steps} calls timed",
                   "eager_us_per_call": round(eager_ms * 1e3, 3),
                   "eager_preallocated_us_per_call": round(eager_dps_ms * 1e3, 3),
                   "cold_cache": cold,
                   "launches_per_call": 1 if one_launch else 2,
                   "dominant_kernel_us": round(ms_dom * 1e3, 3),
                   "merge_and_gaps_us": round((ms - ms_dom) * 1e3, 3)},
        "roofline": roofline,
        "other_roofline": other,
    }


def measure_indexer(steps, warmup):
    """cfg5: the lightning indexer + top-k (block-table slots) and the whole
    indexer -> attention pipeline; returns (fields, workload).  The K operand
    planes are prepared once beforehand (prepare_k: the K cache changes only
    where tokens are appended) for the steady-state figures; the same calls
    deriving them from the raw K every time are timed beside them."""
    from dsa_amd import kernel, prepare_k, workloads
    from dsa_amd.indexer_kernel import run_indexer_and_topk

    d = workloads.cfg5()
    g = workloads.to_device(d, "cuda:0")
    T, Hi, D = d["q_idx"].shape
    S = d["k_idx"].shape[0]
    K = int(d["topk"])
    planes = prepare_k(g["k_idx"], g["k_scale"])
    ia = (g["q_idx"], g["k_idx"], g["k_scale"], g["weights"], g["causal_limit"])
    ip = (g["q_idx"], None, None, g["weights"], g["causal_limit"])
    attn = (g["q_nope"], g["q_pe"], g["ckv_cache"], g["kpe_cache"])

    def indexer():
        run_indexer_and_topk(*ip, K, block_table=g["block_table"], page_size=64, k_planes=planes)

    def indexer_k_prep():
        run_indexer_and_topk(*ia, K, block_table=g["block_table"], page_size=64)

    def scores_only():
        run_indexer_and_topk(*ip, 0, return_scores=True, k_planes=planes)

    def scores_k_prep():
        run_indexer_and_topk(*ia, 0, return_scores=True)

    def k_prep():
        prepare_k(g["k_idx"], g["k_scale"], planes=planes)

    def pipeline():
        sl = run_indexer_and_topk(*ip, K, block_table=g["block_table"], page_size=64,
                                  k_planes=planes)
        kernel(*attn, sl, d["sm_scale"])

    per_graph = min(GRAPH_CALLS, steps)
    ms_idx, timed = time_graph(indexer, steps, warmup)
    ms_idx_kp, _ = time_graph(indexer_k_prep, steps, warmup)
    ms_score, _ = time_graph(scores_only, steps, warmup)
    ms_score_kp, _ = time_graph(scores_k_prep, steps, warmup)
    ms_prep, _ = time_graph(k_prep, steps, warmup)
    ms_pipe, _ = time_graph(pipeline, steps, warmup)
    eager_ms = time_eager(pipeline, steps)
    ops = 2 * T * Hi * S * D                          # algorithmic dot-product ops
    tops = ops / (ms_score * 1e-3) / 1e12
    fields = {
        "us": ms_pipe * 1e3, "ms": ms_pipe, "timed": timed,
        "config": {"workload": f"cfg5: indexer T={T} heads={Hi} dim={D} positions={S} "
                               f"top-{K} -> block-table slots -> cfg2 attention H=16",
                   "timing": f"HIP graphs of {per_graph} back-to-back calls, replayed "
                             f"(plus one graph of the remainder): {steps} calls timed",
                   "k_planes": "prepared once beforehand (prepare_k); *_with_k_prep_us: the "
                               "same call deriving them from the raw K itself",
                   "indexer_topk_us": round(ms_idx * 1e3, 3),
                   "indexer_topk_with_k_prep_us": round(ms_idx_kp * 1e3, 3),
                   "score_kernels_us": round(ms_score * 1e3, 3),
                   "score_kernels_with_k_prep_us": round(ms_score_kp * 1e3, 3),
                   "topk_kernel_us": round((ms_idx - ms_score) * 1e3, 3),
                   "k_prep_us": round(ms_prep * 1e3, 3),
                   "attention_us": round((ms_pipe - ms_idx) * 1e3, 3),
                   "eager_pipeline_us": round(eager_ms * 1e3, 3)},
        "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4),
                     "traffic": load_traffic("cfg5"), "counters": load_counters("cfg5"),
                     "algorithmic_ops": ops,
                     "kernel": "dsa_idx_score_kernel (timed via dsa_indexer_topk with topk=0 "
                               "and prepared K planes; the q operands are derived inside it)"},
    }
    return fields, d


def summary(f):
    """The compact form of a workload's figures carried in the default line."""
    out = {"us_per_call": round(f["us"], 3), "roofline": f["roofline"]}
    if "other_roofline" in f:
        out["other_roofline"] = {k: f["other_roofline"][k]
                                 for k in ("bound", "achieved", "unit", "frac")}
    out["config"] = f["config"]
    return out


def line_of(f, metric, steps, warmup, dtype, data):
    return {"metric": metric, "value": round(f["us"], 3), "unit": "µs/call", "n_gpus": 1,
            "steps": f["timed"], "warmup": warmup, "ms_per_step": round(f["ms"], 6),
            "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
            "data": data, "config": f["config"], "roofline": f["roofline"],
            **({"other_roofline": f["other_roofline"]} if "other_roofline" in f else {})}


ATTN_DATA = "synthetic (seeded; q~N(0,1), cache~N(0,0.5), distinct slots per token)"
IDX_DATA = "synthetic (seeded; q_idx,k_idx ~N(0,1) as e4m3, scale~U(0.5,2), w~N(0,1/8))"


# ---- rocprofv3 records ------------------------------------------------------

PROFILE_STEPS = ["--steps", "40", "--warmup", "5", "--no-cpu-baseline", "--cold-copies", "0"]
COUNTER_PASSES = (("FETCH_SIZE",), ("WRITE_SIZE",),
                  ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CU_CYCLES", "SQ_INSTS_MFMA"),
                  ("TCC_HIT_sum", "TCC_MISS_sum"),
                  ("SQ_LDS_IDX_ACTIVE", "SQ_LDS_BANK_CONFLICT"))
CALIBRATION_BYTES = 1 << 28


def _short_name(name: str) -> str:
    """Kernel name without namespaces and parameter list."""
    base = name.replace("(anonymous namespace)::", "").replace("void ", "").replace("dsa::", "")
    return base.split("(")[0].strip()


def _dominant(config: str, names):
    """The kernel of a workload's measured launch: for attention the
    gather-attention kernel (not the merge kernel), for cfg5 the score kernel
    (the timed score step, which reads prepared K planes and derives the q
    operands itself)."""
    if config == "cfg5":
        return [n for n in names if "dsa_idx_score" in n][:1]
    return [n for n in names if n.startswith("dsa_attn_") and "combine" not in n][:1]


def _rocprof(args, out_dir, tag, program, log):
    """One rocprofv3 run (its own process, under its own time limit); the
    program follows ``--``."""
    cmd = ["timeout", "-s", "KILL", "180", "rocprofv3", *args, "-d", os.path.join(out_dir, tag),
           "-o", "run", "--output-format", "csv", "--", *program]
    print(f"record: {tag}: {' '.join(cmd)}", flush=True)
    env = dict(os.environ, TMPDIR="/tmp")
    with open(log, "w") as f:
        r = subprocess.run(cmd, stdout=f, stderr=subprocess.STDOUT, cwd="/tmp", env=env)
    if r.returncode != 0:
        raise SystemExit(f"record: {tag} failed with status {r.returncode} (log {log})")
    shown = ["python3", "bench.py"] + list(program[2:])
    return " ".join(["rocprofv3", *args, "-d <out> -o run --output-format csv --", *shown])


def _counters(path):
    """{kernel: {counter: median over dispatches}} of a counter pass (values of
    one dispatch summed over the counter's instances)."""
    import collections
    import csv
    import statistics
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    with open(path) as f:
        for r in csv.DictReader(f):
            per[(r["Dispatch_Id"], _short_name(r["Kernel_Name"]))][r["Counter_Name"]] += \
                float(r["Counter_Value"])
    agg = collections.defaultdict(lambda: collections.defaultdict(list))
    for (_, k), v in per.items():
        for c, x in v.items():
            agg[k][c].append(x)
    return {k: {c: statistics.median(v) for c, v in d.items()} for k, d in agg.items()}


def record_profiles(out_dir: str, configs, profiles_dir: str) -> None:
    """Runs the profiler over every workload and writes
    <profiles_dir>/traffic.json and <profiles_dir>/<kernel>_<workload>.txt
    from what it measured (an existing traffic.json there is updated)."""
    import csv
    out_dir = os.path.abspath(out_dir)
    os.makedirs(out_dir, exist_ok=True)
    os.makedirs(profiles_dir, exist_ok=True)
    bench = [sys.executable, os.path.join(ROOT, "bench.py")]
    calib = {}
    cal_cmds = []
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        tag = f"pmc_{ctr}_copy"
        cal_cmds.append(_rocprof(["--pmc", ctr], out_dir, tag,
                                 bench + ["--copy-calibration", str(CALIBRATION_BYTES)],
                                 os.path.join(out_dir, tag + ".log")))
        vals = _counters(os.path.join(out_dir, tag, "run_counter_collection.csv"))
        kib = max(v.get(ctr, 0.0) for k, v in vals.items() if "copy" in k.lower())
        calib[ctr] = (CALIBRATION_BYTES / 1024.0) / kib  # KiB per KiB the counter reads
    cal_note = (f"FETCH_SIZE x{calib['FETCH_SIZE']:.4f}, WRITE_SIZE x{calib['WRITE_SIZE']:.4f} "
                f"(plain device copy of {CALIBRATION_BYTES} bytes)")
    path = os.path.join(profiles_dir, "traffic.json")
    try:
        with open(path) as f:
            table = json.load(f)
    except (OSError, ValueError):
        table = {}
    digest = csrc_hash()
    for c in configs:
        program = bench + PROFILE_STEPS + ["--config", c]
        cmds = [_rocprof(["--kernel-trace", "--stats"], out_dir, f"trace_{c}", program,
                         os.path.join(out_dir, f"trace_{c}.log"))]
        stats = []
        with open(os.path.join(out_dir, f"trace_{c}", "run_kernel_stats.csv")) as f:
            for r in csv.DictReader(f):
                stats.append((_short_name(r["Name"]), int(r["Calls"]), float(r["AverageNs"]) / 1e3,
                              float(r["MinNs"]) / 1e3, float(r["MaxNs"]) / 1e3,
                              float(r["Percentage"])))
        dom = _dominant(c, [n for n, *_ in stats])
        ctr = {}
        for group in COUNTER_PASSES:
            tag = f"pmc_{group[0]}_{c}"
            cmds.append(_rocprof(["--pmc", *group], out_dir, tag, program,
                                 os.path.join(out_dir, tag + ".log")))
            vals = _counters(os.path.join(out_dir, tag, "run_counter_collection.csv"))
            for k in dom:
                for name, x in vals.get(k, {}).items():
                    ctr[name] = ctr.get(name, 0.0) + x
        fetch = ctr.get("FETCH_SIZE", 0.0) * 1024 * calib["FETCH_SIZE"]
        write = ctr.get("WRITE_SIZE", 0.0) * 1024 * calib["WRITE_SIZE"]
        busy = ctr.get("SQ_BUSY_CU_CYCLES", 0.0)
        mfma = ctr.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (4 * busy) if busy else None
        hits, miss = ctr.get("TCC_HIT_sum", 0.0), ctr.get("TCC_MISS_sum", 0.0)
        # LDS cycles summed over the CUs, against the CUs' busy cycles; bank
        # conflicts as a share of the LDS cycles
        lds_active = ctr.get("SQ_LDS_IDX_ACTIVE", 0.0)
        lds = lds_active / busy if busy else None
        ldsc = ctr.get("SQ_LDS_BANK_CONFLICT", 0.0) / lds_active if lds_active else None
        name = dom[-1] if dom else "none"
        summary_file = f"{name.split('<')[0]}_{c}.txt"
        dur = {n: avg for n, _, avg, *_ in stats}
        table[c] = {
            "kernel": " + ".join(dom),
            "kernel_avg_us": round(sum(dur.get(k, 0.0) for k in dom), 3),
            "fetch_bytes_per_launch": int(round(fetch)),
            "write_bytes_per_launch": int(round(write)),
            "hbm_bytes_per_launch": int(round(fetch + write)),
            "mfma_busy_frac": round(mfma, 4) if mfma is not None else None,
            "l2_hit_frac": round(hits / (hits + miss), 4) if hits + miss else None,
            "lds_busy_frac": round(lds, 4) if lds is not None else None,
            "lds_bank_conflict_frac": round(ldsc, 4) if ldsc is not None else None,
            "calibration": cal_note,
            "csrc_sha256": digest,
            "source": f"profiles/{summary_file}",
        }
        lines = [f"rocprofv3 record of workload {c}: dominant launch {' + '.join(dom)}",
                 f"kernel sources sha256 {digest} (bench.py csrc_hash)", "",
                 "Commands (each its own run, from /tmp with TMPDIR=/tmp):"]
        lines += [f"  {x}" for x in cmds + cal_cmds]
        lines += ["", "Kernel trace (--kernel-trace --stats): calls, average / min / max us, share"]
        for n, calls, avg, mn, mx, pct in stats:
            if pct >= 0.5:
                lines.append(f"  {n:70s} {calls:6d} {avg:10.3f} {mn:10.3f} {mx:10.3f} {pct:6.1f}%")
        lines += ["", "Counters of the dominant launch (median per dispatch, summed over its "
                      "kernels):"]
        lines += [f"  {k:28s} {v:.6g}" for k, v in sorted(ctr.items())]
        lines += ["", f"Calibration: {cal_note}",
                  f"HBM bytes per launch: fetched {fetch:,.0f} + written {write:,.0f} = "
                  f"{fetch + write:,.0f}",
                  f"MFMA busy (SQ_VALU_MFMA_BUSY_CYCLES / (4 x SQ_BUSY_CU_CYCLES)): "
                  + (f"{mfma:.4f}" if mfma is not None else "n/a"),
                  "L2 hit (TCC_HIT / (TCC_HIT + TCC_MISS)): "
                  + (f"{hits / (hits + miss):.4f}" if hits + miss else "n/a"),
                  "LDS busy (SQ_LDS_IDX_ACTIVE / SQ_BUSY_CU_CYCLES): "
                  + (f"{lds:.4f}" if lds is not None else "n/a")
                  + "; bank-conflict share of LDS cycles (SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE): "
                  + (f"{ldsc:.4f}" if ldsc is not None else "n/a")]
        with open(os.path.join(profiles_dir, summary_file), "w") as f:
            f.write("\n".join(lines) + "\n")
        with open(path, "w") as f:
            json.dump(table, f, indent=1)
            f.write("\n")
        print(f"record: {c}: {table[c]}", flush=True)


def main():
    a = parse()
    if a.copy_calibration:
        copy_calibration(a.copy_calibration)
        return
    if a.record_profiles:
        record_profiles(a.record_profiles, [c for c in a.profile_configs.split(",") if c],
                        a.profiles_dir)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for {max(a.gpus, world)}); "
              "the DSA path shards by tokens/heads with no exchange and is benchmarked at N=1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from dsa_amd import workloads
    torch.cuda.set_device(0)

    if a.config == "cfg5":
        f, d = measure_indexer(a.steps, a.warmup)
        line = line_of(f, "µs/call, lightning indexer + top-k -> DSA attention (cfg5)", a.steps,
                       a.warmup, "fp8-e4m3 scores (exact), bf16 attention", IDX_DATA)
        if not a.no_cpu_baseline:
            line["cpu_baseline"] = cpu_indexer_baseline(d)
        print(json.dumps(line), flush=True)
        return

    name = a.config or "cfg2"
    d = workloads.CONFIGS[name]()
    cold = a.cold_copies if a.cold_copies >= 0 else COLD_COPIES.get(name, 0)
    f = measure_attention(name, d, a.steps, a.warmup, cold)
    T, H, _ = d["q_nope"].shape
    K = d["sparse_indices"].shape[1]
    metric = METRIC if name == "cfg2" else \
        f"µs/call + HBM GB/s & MFMA %, DSA sparse attention H={H} topk={K} T={T} ({name})"
    line = line_of(f, metric, a.steps, a.warmup, "bf16", ATTN_DATA)
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(d)
    del d
    if a.config is None:
        # every other workload, timed in this same run
        steps = min(a.steps, EXTRA_STEPS)
        warm = min(a.warmup, 10)
        extra = {}
        for other in ("cfg1", "cfg3", "cfg4", "t1"):
            od = workloads.CONFIGS[other]()
            # cfg4's 75.5 MB cache also fits the Infinity Cache: 4 copies (302 MB) rotate
            extra[other] = summary(measure_attention(other, od, steps, warm,
                                                     COLD_COPIES.get(other, 0)))
            if not a.no_cpu_baseline:
                extra[other]["cpu_baseline"] = cpu_baseline(od)
            del od
            torch.cuda.empty_cache()
        extra["t1"]["reference_published"] = T1_REFERENCE
        fi, di = measure_indexer(steps, warm)
        extra["cfg5"] = summary(fi)
        if not a.no_cpu_baseline:
            extra["cfg5"]["cpu_baseline"] = cpu_indexer_baseline(di)
        line["workloads"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

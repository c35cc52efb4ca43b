#!/usr/bin/env python3
"""Benchmark the RPA hot path on one MI355X; prints ONE JSON line.

A step is one ragged_paged_attention call over one synthetic batch of the
chosen configuration (default C2: 64-seq bf16 GQA decode, the configuration
BASELINE.json's metric is quoted on).  Inputs are resident in HBM before the
clock starts; K/V pools are rotated between calls so every call streams its KV
from HBM (the 256 MB Infinity Cache never holds the next call's pages).

value      = algorithmic KV bytes per step / measured step time (SI GB/s)
roofline   = (KV + Q + O bytes) / average duration of the attention kernel,
             timed with HIP events recorded around that kernel alone in every
             timed step (timing-only events: no system-scope fence), against
             MI355X's 8 TB/s HBM peak (or the bf16 MFMA peak for prefill rows)
cpu_baseline = the numpy oracle (oracle/rpa_oracle.py) on a bounded sample of
             the same configuration, on every core of this process's affinity set (BLAS
             threads matched), median of 3 runs.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT), str(ROOT / "tpu-cake_amd")]

METRIC = "RPA decode KV-read GB/s (% of HBM peak) + tokens/s, 64-seq bf16 GQA, 1 GPU"
# configurations beyond BASELINE's five: C2 with the 512-key sliding window of Inkling's largest
# decode family (RPAd-...-sw_512), whose algorithmic bytes are the windows' keys only
# (tpu_cake_amd.workloads.WINDOWED_CONFIGS)


def _rates():
    from tpu_cake_amd.cost_model import mi355x_rates

    return mi355x_rates()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _cores() -> int:
    """Threads for the CPU baseline: the cores of this process's affinity set, capped by
    OMP_NUM_THREADS when the host sets a smaller CPU share that way."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    return min(n, int(omp)) if omp.isdigit() and int(omp) > 0 else n


def cpu_baseline(case, budget_s: float = 18.0, runs: int = 3, sliding_window=None) -> dict:
    """The oracle (oracle/rpa_oracle.py, a numpy restatement of ref_ragged_paged_attention) timed on
    this host: every core of the affinity set, BLAS threads set to match, on the first sequences of
    the same workload sized to about budget_s over ``runs`` runs; the median run is reported."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import rpa_oracle as orc

    n = int(case.num_seqs[0])
    cores = _cores()
    kw = dict(sm_scale=case.sm_scale, kv_scales=case.kv_scales, kv_dtype=case.kv_dtype, sliding_window=sliding_window)

    def run(k):
        t0 = time.perf_counter()
        orc.ref_ragged_paged_attention(case.q, case.kv_pages, case.kv_lens, case.page_indices, case.cu_q_lens,
                                       np.array([k], np.int32), **kw)
        return time.perf_counter() - t0

    with threadpool_limits(limits=cores):
        per_seq = run(1)  # also warms the BLAS pool
        # size the sample: grow k while the estimate stays within one run's share of the budget
        k, t_k = 1, per_seq
        while k < n and t_k < budget_s / runs / 2:
            k = min(n, 2 * k)
            t_k = run(k)
        times = sorted(run(k) for _ in range(runs))
    dt = times[len(times) // 2]
    from tpu_cake_amd.cost_model import rpa_work

    w = case.work(sliding_window)
    part = rpa_work(case.kv_lens[:k], np.diff(case.cu_q_lens[: k + 1]), num_q_heads=case.num_q_heads,
                    num_kv_heads=case.num_kv_heads, head_dim=case.head_dim, page_size=case.page_size,
                    kv_dtype=case.kv_dtype, sliding_window=sliding_window)
    kv_bytes = part.kv_read_bytes + part.scale_bytes
    q_toks = int(case.cu_q_lens[k] - case.cu_q_lens[0])
    return {
        "value": round(kv_bytes / dt / 1e9, 4),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "tokens_per_s": round(q_toks / dt, 2),
        "seconds": round(dt, 3),
        "runs_s": [round(t, 3) for t in times],
        "blas_threads": cores,
        "affinity_cores": len(os.sched_getaffinity(0)),
        "sample": (f"first {k} of {n} sequences ({part.keys_read} KV tokens read, {q_toks} query tokens; "
                   f"{kv_bytes / max(w.kv_read_bytes + w.scale_bytes, 1):.1%} of the step's KV bytes), "
                   f"median of {runs} runs on {cores} cores"),
    }


def copy_probe_gbps(dev, nbytes: int = 1 << 30, reps: int = 5) -> float:
    """Achieved bandwidth of torch's device-to-device copy (bytes read + written / time) on this box,
    reported beside the 8 TB/s published peak (a copy kernel, not a bound on a read stream)."""
    import torch

    src = torch.empty(nbytes // 4, dtype=torch.int32, device=dev).fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    sec = a.elapsed_time(b) / 1e3 / reps
    del src, dst
    return 2 * nbytes / sec / 1e9


def kernel_source_digest() -> str:
    """sha256[:16] of the kernel sources with comments and blank space removed (so that editing
    a comment does not orphan a measurement); tpu_cake_amd.evidence.kernel_source_digest."""
    from tpu_cake_amd.evidence import kernel_source_digest as digest

    return digest()


def measured_traffic(cfg: str):
    """HBM bytes per attention-kernel dispatch (for "inkling": per step, all three kernels) from
    the committed rocprofv3 PMC summary (profiles/pmc_traffic.json: FETCH_SIZE and WRITE_SIZE,
    each scaled by the same counter's reading for a 1 GiB copy), used only if it was measured on
    the current kernel sources."""
    path = ROOT / "profiles" / "pmc_traffic.json"
    if not path.exists():
        return None
    data = json.loads(path.read_text())
    if kernel_source_digest() != data.get("source_sha256_16") or cfg not in data.get("configs", {}):
        return None
    return data["configs"][cfg]["traffic_bytes"]


def fused_cpu_baseline(case, budget_s: float = 18.0, runs: int = 3) -> dict:
    """The fused-decode oracle (oracle/rpa_fused_oracle.py) on the first sequences of the step, on
    every core of the affinity set (BLAS threads matched), median of ``runs`` runs."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import rpa_fused_oracle as fo

    a = case.arrays
    n = len(a["kv_lengths"])
    S = a["cache"].shape[1]
    cores = _cores()

    def subset(k):
        pages = int(a["cu_kv_lens"][k]) // S
        sub = dict(a)
        for key in ("queries", "keys", "values", "kv_lengths", "relative_states"):
            sub[key] = a[key][:k]
        sub["cu_kv_lens"] = a["cu_kv_lens"][: k + 1]
        sub["cu_q_lens"] = np.arange(k + 1, dtype=np.int32)
        sub["distribution"] = np.full((3,), k, dtype=np.int32)
        sub["page_indices"] = a["page_indices"][:pages]
        sub["cache"] = a["cache"].reshape(a["cache"].shape[0], S, -1, 2, a["cache"].shape[-1])
        return sub

    def run(k):
        sub = subset(k)
        t0 = time.perf_counter()
        fo.inkling_fused_rpa_reference(sub)
        return time.perf_counter() - t0

    with threadpool_limits(limits=cores):
        k, t_k = 1, run(1)
        while k < n and t_k < budget_s / runs / 2:
            k = min(n, 2 * k)
            t_k = run(k)
        times = sorted(run(k) for _ in range(runs))
    dt = times[len(times) // 2]
    toks = int(a["kv_lengths"][:k].sum())
    kv_bytes = toks * a["keys"].shape[1] * 2 * 128 * 2
    return {"value": round(kv_bytes / dt / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "tokens_per_s": round(k / dt, 2), "seconds": round(dt, 3), "runs_s": [round(t, 3) for t in times],
            "blas_threads": cores,
            "sample": f"first {k} of {n} sequences ({toks} KV tokens, {k} decode steps) of the same step, "
                      f"median of {runs} runs on {cores} cores"}


def fused_bench(args, dev) -> int:
    """One step = one fused Inkling decode call (cache write + prep + attention + combine)."""
    import numpy as np
    import torch

    from tpu_cake_amd import fused
    from tpu_cake_amd.workloads import FUSED_DESCRIPTION, make_fused_case

    t0 = time.perf_counter()
    page = args.fused_page_size
    case = make_fused_case(seed=args.seed if args.seed is not None else 102, page_size=page)
    log(f"built inkling in {time.perf_counter() - t0:.1f}s")
    a = case.arrays
    tensors = []
    for name in fused.INPUT_NAMES:
        x = a[name]
        t = torch.from_numpy(x.view(np.int16).copy()).view(torch.bfloat16) if x.dtype == np.uint16 else \
            torch.from_numpy(np.ascontiguousarray(x))
        tensors.append(t.to(dev))
    fused.preflight(*tensors)  # the reference's run_preflighted check, once per metadata layout
    cache_bytes = tensors[3].numel() * 2
    copies = max(2, math.ceil(args.rotate_bytes / cache_bytes))
    caches = [tensors[3]] + [tensors[3].clone() for _ in range(copies - 1)]
    S = tensors[3].shape[1]
    pps = int(((a["kv_lengths"].astype(np.int64) + S - 1) // S).max())
    out = torch.empty_like(tensors[0])

    def call(i):
        xs = list(tensors)
        xs[3] = caches[i % copies]
        fused.invoke(*xs, sm_scale=case.sm_scale, pages_per_seq=pps, out=out)

    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    start.record()
    for i in range(args.steps):
        call(i)
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = start.elapsed_time(stop) / args.steps
    nseq, hq = a["queries"].shape[:2]
    kv_bytes = case.kv_read_bytes()
    moved = kv_bytes + 2 * nseq * hq * 128 * 2 + 2 * a["keys"].size * 2 * 2
    peak = _rates().hbm_bytes_per_second / 1e9
    value = kv_bytes / (ms_step * 1e-3) / 1e9
    achieved = moved / (ms_step * 1e-3) / 1e9
    result = {
        "metric": "Inkling fused decode KV-read GB/s (% of HBM peak) + tokens/s, 64-seq bf16 GQA, 1 GPU",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic: seeded N(0,1) queries / new K,V, N(0,0.25) cache, N(0,0.4) relative tensors",
        "config": {"workload": "inkling: " + FUSED_DESCRIPTION.replace("page 64", f"page {page}"), "num_seqs": int(nseq),
                   "sum_kv_len": int(a["kv_lengths"].sum()), "kv_bytes_per_step": kv_bytes,
                   "cache_copies_rotated": copies},
        "tokens_per_s": round(nseq / (ms_step * 1e-3), 1),
        "hbm_fraction": round(value / peak, 4),
        "wall_s_timed_region": round(wall, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": peak, "unit": "GB/s",
                     "frac": round(achieved / peak, 4),
                     "traffic": measured_traffic("inkling") if page == 64 else None,
                     "basis": "whole step (every launch of the call: attention with the in-kernel bias, merge "
                              "with the new-token store; a preparation launch first for shapes that need one)"},
    }
    if not args.no_cpu_baseline:
        log("cpu baseline (fused oracle) ...")
        result["cpu_baseline"] = fused_cpu_baseline(case)
    print(json.dumps(result), flush=True)
    return 0


def host_submit(args, dev, calls: int = 400) -> int:
    """Host time per call: ``calls`` back-to-back ops.ragged_paged_attention calls on C1 (kernels of
    a few microseconds, so the host is the bound), wall time / calls, median of 5 batches; the
    same with the validation plan dropped each call (the first call of a new signature); the call
    prepared once (ops.PreparedCall); the call captured into a HIP graph (ops.CapturedCall), per
    replay; and 32 calls captured into one graph (ops.CapturedCalls), per call."""
    import statistics

    import torch

    from tpu_cake_amd import ops
    from tpu_cake_amd.workloads import make_config

    case = make_config("c1", seed=args.seed)
    d = ops.case_to_device(case, dev)
    out = torch.empty_like(d["q"])

    def call():
        ops.ragged_paged_attention(d["q"], d["kv_pages"], d["kv_lens"], d["page_indices"], d["cu_q_lens"],
                                   d["num_seqs"], sm_scale=case.sm_scale, out=out)

    for _ in range(20):
        call()
    torch.cuda.synchronize()
    res = {}
    for label, cold in (("cached_plan", False), ("plan_each_call", True)):
        per = []
        for _ in range(5):
            t0 = time.perf_counter()
            for _ in range(calls):
                if cold:
                    ops._plans.clear()
                call()
            per.append((time.perf_counter() - t0) / calls * 1e6)
            torch.cuda.synchronize()
        res[label] = round(statistics.median(per), 2)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(calls):
        call()
    ev1.record()
    torch.cuda.synchronize()
    device_us = round(ev0.elapsed_time(ev1) * 1e3 / calls, 2)
    # the same call prepared once (ops.PreparedCall: one foreign call per step)
    pc = ops.PreparedCall(d["q"], d["kv_pages"], d["kv_lens"], d["page_indices"], d["cu_q_lens"], d["num_seqs"],
                          sm_scale=case.sm_scale, out=torch.empty_like(d["q"]))
    for _ in range(20):
        pc()
    torch.cuda.synchronize()
    per = []
    for _ in range(5):
        t0 = time.perf_counter()
        for _ in range(calls):
            pc()
        per.append((time.perf_counter() - t0) / calls * 1e6)
        torch.cuda.synchronize()
    res["prepared_call"] = round(statistics.median(per), 2)
    # the same call captured into a HIP graph and replayed (ops.CapturedCall)
    cc = ops.CapturedCall(d["q"], d["kv_pages"], d["kv_lens"], d["page_indices"], d["cu_q_lens"], d["num_seqs"],
                          sm_scale=case.sm_scale, out=torch.empty_like(d["q"]))
    for _ in range(20):
        cc.replay()
    torch.cuda.synchronize()
    per = []
    for _ in range(5):
        t0 = time.perf_counter()
        for _ in range(calls):
            cc.replay()
        per.append((time.perf_counter() - t0) / calls * 1e6)
        torch.cuda.synchronize()
    res["graph_replay"] = round(statistics.median(per), 2)
    ev0.record()
    for _ in range(calls):
        cc.replay()
    ev1.record()
    torch.cuda.synchronize()
    graph1_us = round(ev0.elapsed_time(ev1) * 1e3 / calls, 2)
    # a whole step's calls in one graph (ops.CapturedCalls: 32 calls, one per layer of a model,
    # here over the same buffers), per call
    layers = 32
    many = ops.CapturedCalls([((d["q"], d["kv_pages"], d["kv_lens"], d["page_indices"], d["cu_q_lens"],
                                d["num_seqs"]), dict(sm_scale=case.sm_scale, out=torch.empty_like(d["q"])))
                              for _ in range(layers)])
    for _ in range(5):
        many.replay()
    torch.cuda.synchronize()
    reps = max(1, calls // layers)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(reps):
        many.replay()
    ev1.record()
    res["graph_of_32_calls"] = round((time.perf_counter() - t0) / (reps * layers) * 1e6, 2)
    torch.cuda.synchronize()
    print(json.dumps({"host_submit_us_per_call": res, "device_us_per_call_back_to_back": device_us,
                      "device_us_per_call_graph_replays": graph1_us,
                      "device_us_per_call_graph_of_32_calls": round(ev0.elapsed_time(ev1) * 1e3 / (reps * layers), 2),
                      "calls": calls, "workload": "c1 (kernels of a few us: the host is the bound)"}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5", "c2w", "c3f", "c5t", "c2d64", "c2d256", "inkling"],
                    help="c1..c5: the RPA operator configurations; c2w: C2 with a 512-key sliding window; "
                         "c3f: C3's batch over an fp8 pool; c5t: C5 with one 131072-key sequence; c2d64 / c2d256: C2 at head_dim 64 / 256; "
                         "inkling: the fused decode step (KV-cache write + relative-bias attention)")
    ap.add_argument("--seed", type=int, default=None)
    ap.add_argument("--fused-page-size", type=int, default=64,
                    help="inkling: the cache's page size (64: the profiled workload; any size runs in one "
                         "attention launch)")
    ap.add_argument("--rotate-bytes", type=float, default=2.0e9,
                    help="KV pool copies rotated so that at least this many bytes separate reuses")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--waves-per-cu", type=int, default=None, help="schedule knob (default: the tuned table)")
    ap.add_argument("--prefill-tiles", type=int, default=None, choices=[-1, 0, 1, 2, 3],
                    help="1: prefill kernel, 2: the attention kernel's own prefill tiles, 3: those tiles in "
                         "one 8-wave workgroup per CU, -1: stream-K rows (default: the tuned table)")
    ap.add_argument("--prefill-cost", type=float, default=None, help="schedule knob (default: the tuned table)")
    ap.add_argument("--graph", action="store_true",
                    help="time steps as replays of one-call HIP graphs (ops.CapturedCall, one per rotated pool) "
                         "instead of eager calls")
    ap.add_argument("--host-submit", action="store_true",
                    help="instead of the benchmark, measure the host time to submit one call (C1 shapes, "
                         "calls back to back, no synchronisation in between) and exit")
    ap.add_argument("--copy-probe", type=float, default=0.0, metavar="BYTES",
                    help="instead of the benchmark, run 5 device-to-device copies of BYTES (the known-size "
                         "kernel that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (single-GPU RPA hot path; "
              "multi-GPU sharding is a design note, not built); run with --gpus 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from tpu_cake_amd import ops
    from tpu_cake_amd.timing import KernelEvent
    from tpu_cake_amd.workloads import CONFIG_DESCRIPTIONS, make_config

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    if args.copy_probe:
        n = int(args.copy_probe) // 16 * 16
        gbps = copy_probe_gbps(dev, n)
        print(json.dumps({"copy_probe_bytes": n, "copies": 6, "achieved_gbps": round(gbps, 1)}))
        return 0

    if args.host_submit:
        return host_submit(args, dev)

    if args.config == "inkling":
        return fused_bench(args, dev)

    from tpu_cake_amd.workloads import WINDOWED_CONFIGS

    base_cfg, window = WINDOWED_CONFIGS.get(args.config, (args.config, None))
    t0 = time.perf_counter()
    case = make_config(base_cfg, seed=args.seed)
    log(f"built {args.config} in {time.perf_counter() - t0:.1f}s")
    d = ops.case_to_device(case, dev)
    kv_scales = d.pop("kv_scales", None)
    pool_bytes = d["kv_pages"].numel() * d["kv_pages"].element_size()
    copies = max(2, math.ceil(args.rotate_bytes / pool_bytes))
    pools = [d["kv_pages"]] + [d["kv_pages"].clone() for _ in range(copies - 1)]
    out = torch.empty_like(d["q"])
    torch.cuda.synchronize()

    n = int(case.num_seqs[0])
    T = int(case.cu_q_lens[n])
    work = case.work(window)  # the work convention (tpu_cake_amd.cost_model.rpa_work)
    kv_bytes = work.kv_read_bytes + work.scale_bytes
    qo_bytes = work.q_bytes + work.o_bytes
    flops = work.prefill_flops
    rates = _rates()
    peak = rates.hbm_bytes_per_second / 1e9

    knobs = {k: v for k, v in (("waves_per_cu", args.waves_per_cu), ("prefill_tiles", args.prefill_tiles),
                               ("prefill_cost", args.prefill_cost)) if v is not None}

    def call(i, ev=None):
        ops.ragged_paged_attention(d["q"], pools[i % copies], d["kv_lens"], d["page_indices"], d["cu_q_lens"],
                                   d["num_seqs"], sm_scale=case.sm_scale, kv_scales=kv_scales, out=out,
                                   kernel_events=ev, sliding_window=window, **knobs)

    step = call
    if args.graph:  # one captured call per pool copy, replayed in the pools' rotation
        graphs = [ops.CapturedCall(d["q"], pools[c], d["kv_lens"], d["page_indices"], d["cu_q_lens"], d["num_seqs"],
                                   sm_scale=case.sm_scale, kv_scales=kv_scales, out=out, sliding_window=window,
                                   **knobs) for c in range(copies)]

        def step(i):
            graphs[i % copies].replay()

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # the timed region: K calls and nothing else (the headline value)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    start.record()
    for i in range(args.steps):
        step(i)
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = start.elapsed_time(stop) / args.steps
    # the same K calls again with timing-only HIP events (no system-scope fence at record) around
    # every attention kernel, on its stream: the kernel's duration for the roofline.  The events
    # themselves lengthen a step (recorded between the attention and merge launches), which is
    # why the headline comes from the region above.
    evs = [(KernelEvent(), KernelEvent()) for _ in range(args.steps)]
    start.record()
    for i in range(args.steps):
        call(args.steps + i, evs[i])
    stop.record()
    torch.cuda.synchronize()
    ms_step_events = start.elapsed_time(stop) / args.steps
    kern_ms = [a.elapsed_time(b) for a, b in evs]
    kern_avg = float(np.mean(kern_ms))
    kern_med = float(np.median(kern_ms))
    del pools
    ceiling = copy_probe_gbps(dev)

    value = kv_bytes / (ms_step * 1e-3) / 1e9
    achieved_bw = (kv_bytes + qo_bytes) / (kern_avg * 1e-3) / 1e9
    desc = CONFIG_DESCRIPTIONS[base_cfg] + (f"; sliding_window {window}" if window else "")
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8" if case.kv_dtype == "fp8" else "bf16",
        "data": "synthetic: seeded N(0,1) bf16 q/K/V, page tables a seeded permutation of a 1.25x pool",
        "config": {
            "workload": f"{args.config}: {desc}",
            "num_seqs": n,
            "query_tokens": T,
            "sum_kv_len": int(case.kv_lens[:n].sum()),
            "kv_bytes_per_step": kv_bytes,
            "kv_pool_copies_rotated": copies,
            **({"steps_as": "one-call HIP graph replays"} if args.graph else {}),
            **({"knobs": knobs} if knobs else {}),
        },
        "tokens_per_s": round(T / (ms_step * 1e-3), 1),
        "hbm_fraction": round(value / peak, 4),
        "attn_kernel_ms": {"avg": round(kern_avg, 5), "median": round(kern_med, 5),
                           "p90": round(float(np.percentile(kern_ms, 90)), 5),
                           "ms_per_step_with_kernel_events": round(ms_step_events, 5)},
        "wall_s_timed_region": round(wall, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved_bw, 2), "peak": peak, "unit": "GB/s",
                     "frac": round(achieved_bw / peak, 4), "traffic": measured_traffic(args.config),
                     "copy_probe_gbps": round(ceiling, 1),
                     "basis": "algorithmic KV + Q + O bytes (tpu_cake_amd.cost_model.rpa_work) / average "
                              "rpa_attn_kernel duration (HIP events on its stream, K more calls right after "
                              "the timed region); copy_probe_gbps: torch's 1 GiB device-to-device copy on this "
                              "box, read + write bytes / time"},
    }
    if flops:
        result["prefill_mfma"] = {"flops": flops, "achieved_tflops_over_attn_kernel":
                                  round(flops / (kern_avg * 1e-3) / 1e12, 2),
                                  "peak_tflops": rates.compute_flops_per_second / 1e12}
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle) ...")
        result["cpu_baseline"] = cpu_baseline(case, sliding_window=window)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

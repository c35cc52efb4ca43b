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
             the same configuration, 1 thread, on this host.
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

HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E, AMD published
BF16_PEAK_TFLOPS = 2500.0       # MI355X dense bf16 MFMA, AMD published
METRIC = "RPA decode KV-read GB/s (% of HBM peak) + tokens/s, 64-seq bf16 GQA, 1 GPU"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(case, budget_s: float = 20.0) -> dict:
    """Time the oracle on the first sequences of the workload (about budget_s of work)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import rpa_oracle as orc

    n = int(case.num_seqs[0])
    lens = case.kv_lens[:n].astype(np.int64)
    with threadpool_limits(limits=1):
        # probe speed on one sequence, then size the sample
        t0 = time.perf_counter()
        orc.ref_ragged_paged_attention(case.q, case.kv_pages, case.kv_lens, case.page_indices, case.cu_q_lens,
                                       np.array([1], np.int32), sm_scale=case.sm_scale,
                                       kv_scales=case.kv_scales, kv_dtype=case.kv_dtype)
        probe = max(time.perf_counter() - t0, 1e-3)
        per_tok = probe / max(int(lens[0]), 1)
        k = 1
        while k < n and per_tok * int(lens[: k + 1].sum()) < budget_s:
            k += 1
        t0 = time.perf_counter()
        orc.ref_ragged_paged_attention(case.q, case.kv_pages, case.kv_lens, case.page_indices, case.cu_q_lens,
                                       np.array([k], np.int32), sm_scale=case.sm_scale,
                                       kv_scales=case.kv_scales, kv_dtype=case.kv_dtype)
        dt = time.perf_counter() - t0
    toks = int(lens[:k].sum())
    elem = 1 if case.kv_dtype == "fp8" else 2
    kv_bytes = toks * case.num_kv_heads * 2 * case.head_dim * elem
    q_toks = int(case.cu_q_lens[k] - case.cu_q_lens[0])
    return {
        "value": round(kv_bytes / dt / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "tokens_per_s": round(q_toks / dt, 2),
        "seconds": round(dt, 3),
        "sample": f"first {k} of {n} sequences ({toks} KV tokens, {q_toks} query tokens) of the same workload",
    }


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


def fused_cpu_baseline(case, budget_s: float = 20.0) -> dict:
    """The fused-decode oracle (oracle/rpa_fused_oracle.py) on the first sequences of the step."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import rpa_fused_oracle as fo

    a = case.arrays
    n = len(a["kv_lengths"])
    S = a["cache"].shape[1]

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

    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        fo.inkling_fused_rpa_reference(subset(1))
        per_seq = max(time.perf_counter() - t0, 1e-3) / max(int(a["kv_lengths"][0]), 1)
        k = 1
        while k < n and per_seq * int(a["kv_lengths"][: k + 1].sum()) < budget_s:
            k += 1
        t0 = time.perf_counter()
        fo.inkling_fused_rpa_reference(subset(k))
        dt = time.perf_counter() - t0
    toks = int(a["kv_lengths"][:k].sum())
    kv_bytes = toks * a["keys"].shape[1] * 2 * 128 * 2
    return {"value": round(kv_bytes / dt / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "tokens_per_s": round(k / dt, 2), "seconds": round(dt, 3),
            "sample": f"first {k} of {n} sequences ({toks} KV tokens, {k} decode steps) of the same step"}


def fused_bench(args, dev) -> int:
    """One step = one fused Inkling decode call (cache write + prep + attention + combine)."""
    import numpy as np
    import torch

    from tpu_cake_amd import fused
    from tpu_cake_amd.workloads import FUSED_DESCRIPTION, make_fused_case

    t0 = time.perf_counter()
    case = make_fused_case(seed=args.seed if args.seed is not None else 102)
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
    value = kv_bytes / (ms_step * 1e-3) / 1e9
    achieved = moved / (ms_step * 1e-3) / 1e9
    result = {
        "metric": "Inkling fused decode KV-read GB/s (% of HBM peak) + tokens/s, 64-seq bf16 GQA, 1 GPU",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic: seeded N(0,1) queries / new K,V, N(0,0.25) cache, N(0,0.4) relative tensors",
        "config": {"workload": f"inkling: {FUSED_DESCRIPTION}", "num_seqs": int(nseq),
                   "sum_kv_len": int(a["kv_lengths"].sum()), "kv_bytes_per_step": kv_bytes,
                   "cache_copies_rotated": copies},
        "tokens_per_s": round(nseq / (ms_step * 1e-3), 1),
        "hbm_fraction": round(value / HBM_PEAK_GBPS, 4),
        "wall_s_timed_region": round(wall, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": measured_traffic("inkling"),
                     "basis": "whole step (cache write, metadata and bias-table kernels, attention, combine)"},
    }
    if not args.no_cpu_baseline:
        log("cpu baseline (fused oracle) ...")
        result["cpu_baseline"] = fused_cpu_baseline(case)
    print(json.dumps(result), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5", "inkling"],
                    help="c1..c5: the RPA operator configurations; inkling: the fused decode step "
                         "(KV-cache write + relative-bias attention)")
    ap.add_argument("--seed", type=int, default=None)
    ap.add_argument("--rotate-bytes", type=float, default=2.0e9,
                    help="KV pool copies rotated so that at least this many bytes separate reuses")
    ap.add_argument("--no-cpu-baseline", action="store_true")
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
        src = torch.empty(n // 4, dtype=torch.int32, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "copies": 5}))
        return 0

    if args.config == "inkling":
        return fused_bench(args, dev)

    t0 = time.perf_counter()
    case = make_config(args.config, seed=args.seed)
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
    kv_bytes = case.kv_read_bytes()
    qo_bytes = 2 * T * case.num_q_heads * case.head_dim * 2
    flops = case.prefill_flops()

    def call(i, ev=None):
        ops.ragged_paged_attention(d["q"], pools[i % copies], d["kv_lens"], d["page_indices"], d["cu_q_lens"],
                                   d["num_seqs"], sm_scale=case.sm_scale, kv_scales=kv_scales, out=out,
                                   kernel_events=ev)

    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()
    # timing-only HIP events (no system-scope fence at record) around the attention kernel
    evs = [(KernelEvent(), KernelEvent()) for _ in range(args.steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    start.record()
    for i in range(args.steps):
        call(i, evs[i])
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = start.elapsed_time(stop) / args.steps
    kern_ms = [a.elapsed_time(b) for a, b in evs]
    kern_avg = float(np.mean(kern_ms))
    kern_med = float(np.median(kern_ms))

    value = kv_bytes / (ms_step * 1e-3) / 1e9
    achieved_bw = (kv_bytes + qo_bytes) / (kern_avg * 1e-3) / 1e9
    if flops and args.config == "c3":
        roof_flops = flops / (kern_avg * 1e-3) / 1e12
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
            "workload": f"{args.config}: {CONFIG_DESCRIPTIONS[args.config]}",
            "num_seqs": n,
            "query_tokens": T,
            "sum_kv_len": int(case.kv_lens[:n].sum()),
            "kv_bytes_per_step": kv_bytes,
            "kv_pool_copies_rotated": copies,
        },
        "tokens_per_s": round(T / (ms_step * 1e-3), 1),
        "hbm_fraction": round(value / HBM_PEAK_GBPS, 4),
        "attn_kernel_ms": {"avg": round(kern_avg, 5), "median": round(kern_med, 5),
                           "p90": round(float(np.percentile(kern_ms, 90)), 5)},
        "wall_s_timed_region": round(wall, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved_bw, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved_bw / HBM_PEAK_GBPS, 4), "traffic": None},
    }
    traffic = measured_traffic(args.config)
    if traffic is not None:
        result["roofline"]["traffic"] = traffic
    if flops and args.config == "c3":
        result["prefill_mfma"] = {"flops": flops, "achieved_tflops_over_attn_kernel": round(roof_flops, 2),
                                  "peak_tflops": BF16_PEAK_TFLOPS}
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle) ...")
        result["cpu_baseline"] = cpu_baseline(case)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

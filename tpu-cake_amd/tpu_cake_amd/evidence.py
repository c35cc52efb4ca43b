"""Run evidence for the RPA kernels on MI355X: three-phase runs, profile inspection, receipts.

The reference drives its kernel through a three-phase evidence discipline
(``src/tpu_cake/rpa_bundle.py:664-800``): a *timing* run, a *trace* run and a *counters* run of
the same experiment, each leaving a ``result.json``; an assessment of the captured profiles
against the experiment's expectations (``src/tpu_cake/xprof_evidence.py:286-447``); and a
receipt that accepts the evidence only if every phase ran the same sources on the same inputs,
every artifact is accounted for by role and hash, and every check passed.  This module is that
discipline with MI355X tools:

* timing phase -- HIP timing-only events around the attention kernel (``ops`` ``kernel_events``)
  and around each whole call, plus the caller's correctness check;
* trace phase -- the same steps under ``rocprofv3 --kernel-trace --stats``;
* counters phase -- the same steps under ``rocprofv3 --pmc FETCH_SIZE`` and ``WRITE_SIZE``
  (one counter per pass);
* ``inspect_profile`` -- rocprofv3's CSV output -> per-kernel dispatch statistics and counters,
  assessed against an expectation (required kernels, dispatches per step, counters present);
* ``build_receipt`` / ``validate_receipt`` -- the receipt over the three phases.

The correctness verdict comes from a caller-supplied checker (``run_timing(..., checker=)``: the
call's case and output -> errors and a pass flag); this package ships no reference
implementation, so a receipt without a checked, passing correctness result is rejected.  The
repository's test suite supplies the oracle-backed checker (``tests/evidence_run.py``).

Usage (from the repository root, on a GPU box)::

    python tests/evidence_run.py --config c2 --root OUT            # all phases, oracle checker, receipt
    python -m tpu_cake_amd.evidence inspect OUT/trace               # one profile
    python -m tpu_cake_amd.evidence validate OUT                    # re-check a receipt
"""

from __future__ import annotations

import argparse
import csv
import hashlib
import json
import math
import os
import pathlib
import re
import subprocess
import sys
import time

PACKAGE = pathlib.Path(__file__).resolve().parent
CSRC = PACKAGE.parent / "csrc"
PHASES = ("timing", "trace", "counters")
KERNELS = ("rpa_attn_kernel", "rpa_combine_kernel")
COUNTERS = ("FETCH_SIZE", "WRITE_SIZE")
# MFMA activity of the attention kernel (the reference fails a capture without MXU-busy series,
# src/tpu_cake/xprof_evidence.py:339-349): busy cycles summed over SIMDs, the GPU's active cycles,
# and the bf16 MFMA math ops / 512
MFMA_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE", "SQ_INSTS_VALU_MFMA_MOPS_BF16")


# --------------------------------------------------------------------------- identity
def kernel_source_digest() -> str:
    """sha256[:16] of the kernel sources with comments and blank space removed."""
    text = "".join((CSRC / f).read_text() for f in ("rpa_kernels.hip", "rpa_schedule.h"))
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"\s+", " ", text).strip()
    return hashlib.sha256(text.encode()).hexdigest()[:16]


def sha256_file(path: pathlib.Path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 20), b""):
            h.update(block)
    return h.hexdigest()


def source_identity() -> dict:
    """What a run executed: the kernel sources (comment-insensitive) and the loaded library."""
    from . import _lib

    lib = _lib.library_path()
    return {"kernel_source_digest": kernel_source_digest(),
            "library_sha256": sha256_file(lib) if lib.exists() else None}


# --------------------------------------------------------------------------- profiles
def _kernel_key(name: str) -> str | None:
    for k in ("rpa_attn_kernel", "rpa_prefill_kernel", "rpa_combine_kernel", "rpa_fused_prep_kernel",
              "rpa_inkling_v1_prep_kernel", "rpa_fused_unpad_kernel", "rpa_scratch_clear_kernel",
              "__amd_rocclr_copyBuffer"):
        if k in name:
            return k
    return None


def inspect_profile(path) -> dict:
    """rocprofv3 CSV output under ``path`` -> {kernels: {name: {calls, avg_ns, min_ns, max_ns}},
    counters: {name: {counter: mean per dispatch}}, files: [...]}.  Only this library's kernels
    are reported (by their names); templated instances of one kernel are summed."""
    root = pathlib.Path(path)
    kernels: dict = {}
    counters: dict = {}
    files = sorted(str(p.relative_to(root)) for p in root.rglob("*.csv"))
    for stats in root.rglob("*kernel_stats.csv"):
        for r in csv.DictReader(open(stats)):
            k = _kernel_key(r["Name"])
            if k is None or not k.startswith("rpa"):
                continue
            e = kernels.setdefault(k, {"calls": 0, "total_ns": 0.0, "min_ns": math.inf, "max_ns": 0.0})
            e["calls"] += int(r["Calls"])
            e["total_ns"] += float(r["TotalDurationNs"])
            e["min_ns"] = min(e["min_ns"], float(r["MinNs"]))
            e["max_ns"] = max(e["max_ns"], float(r["MaxNs"]))
    for e in kernels.values():
        e["avg_ns"] = e["total_ns"] / e["calls"] if e["calls"] else 0.0
    dispatches: dict = {}  # counter runs: kernel -> dispatches per counter pass (fewest over passes)
    for cc in root.rglob("*counter_collection.csv"):
        acc: dict = {}
        seen: dict = {}
        for r in csv.DictReader(open(cc)):
            k = _kernel_key(r["Kernel_Name"])
            if k is None or not k.startswith("rpa"):
                continue
            acc.setdefault(k, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
            seen.setdefault(k, set()).add(r.get("Dispatch_Id") or r.get("Correlation_Id"))
        for k, per in acc.items():
            for c, vals in per.items():
                counters.setdefault(k, {})[c] = sum(vals) / len(vals)
        for k, ids in seen.items():
            dispatches[k] = min(dispatches.get(k, len(ids)), len(ids))
    return {"kernels": kernels, "counters": counters, "counter_dispatches": dispatches, "files": files}


def assess_profile(profile: dict, *, dispatches: int, counters: tuple = ()) -> dict:
    """Accept a profile if every kernel of the call was captured at least ``dispatches`` times
    (the timed steps) and, for a counters run, every named counter was read for the attention
    kernel (a counters run names the HBM counters and the MFMA-activity ones)."""
    reasons = []
    for k in KERNELS:
        calls = profile["kernels"].get(k, {}).get("calls", 0)
        if counters:  # a counters run captures dispatches through its counter rows
            calls = profile.get("counter_dispatches", {}).get(k, 0)
        if calls < dispatches:
            reasons.append(f"{k}: {calls} dispatches captured, expected >= {dispatches}")
    for c in counters:
        if c not in profile["counters"].get("rpa_attn_kernel", {}):
            reasons.append(f"rpa_attn_kernel: counter {c} not captured")
    return {"accepted": not reasons, "reasons": reasons}


# --------------------------------------------------------------------------- phases
def _steps(config: str, steps: int, warmup: int, events: bool, seed: int | None = None,
           knobs: dict | None = None) -> dict:
    """Run ``steps`` timed calls of a benchmark configuration (inputs resident, pools rotated);
    with ``events``, time the attention kernel and each whole call with HIP events.  ``knobs``:
    explicit schedule knobs (``waves_per_cu``, ``prefill_tiles``, ``prefill_cost``) for every
    call, else the tuned table's."""
    import torch

    from . import ops
    from .timing import KernelEvent
    from .workloads import make_config

    dev = torch.device("cuda", 0)
    case = make_config(config, seed=seed)
    d = ops.case_to_device(case, dev)
    pool = d["kv_pages"]
    copies = max(2, math.ceil(2e9 / (pool.numel() * pool.element_size())))
    pools = [pool] + [pool.clone() for _ in range(copies - 1)]
    out = torch.empty_like(d["q"])
    kw = dict(sm_scale=case.sm_scale, out=out, **(knobs or {}))
    if "kv_scales" in d:
        kw["kv_scales"] = d["kv_scales"]
    kev = [(KernelEvent(), KernelEvent()) for _ in range(steps)] if events else None
    cev = [(KernelEvent(), KernelEvent()) for _ in range(steps)] if events else None

    def call(i, timed):
        ev = kev[i] if timed and events else None
        if timed and events:
            cev[i][0].record()
        ops.ragged_paged_attention(d["q"], pools[i % copies], d["kv_lens"], d["page_indices"], d["cu_q_lens"],
                                   d["num_seqs"], kernel_events=ev, **kw)
        if timed and events:
            cev[i][1].record()

    for i in range(warmup):
        call(i, False)
    torch.cuda.synchronize()
    for i in range(steps):
        call(i, True)
    torch.cuda.synchronize()
    res = {"config": config, "steps": steps, "warmup": warmup, "seed": seed, "knobs": knobs or {}}
    if events:
        res["attention_ns"] = [round(a.elapsed_time(b) * 1e6) for a, b in kev]
        res["call_ns"] = [round(a.elapsed_time(b) * 1e6) for a, b in cev]
    res["output_sha256"] = hashlib.sha256(out.view(torch.int16).cpu().numpy().tobytes()).hexdigest()
    res["input_sha256"] = hashlib.sha256(case.q.tobytes() + case.kv_pages.tobytes() + case.kv_lens.tobytes()
                                         + case.page_indices.tobytes()).hexdigest()
    return res, case, out


def _write_result(phase_root: pathlib.Path, mode: str, body: dict) -> dict:
    phase_root.mkdir(parents=True, exist_ok=True)
    arts = []
    for p in sorted(phase_root.rglob("*")):
        if p.is_file() and p.name != "result.json":
            arts.append({"path": str(p.relative_to(phase_root)), "sha256": sha256_file(p),
                         "role": "rocprofv3" if p.suffix == ".csv" else "samples"})
    result = {"mode": mode, "identity": source_identity(), **body, "artifacts": arts}
    (phase_root / "result.json").write_text(json.dumps(result, indent=1, sort_keys=True) + "\n")
    return result


def run_timing(root, config: str, steps: int, warmup: int, checker=None) -> dict:
    """The timing phase; ``checker(case, out) -> dict`` with at least ``passed`` (the reference's
    correctness gate, rpa_runner.py:105-122) supplies the correctness verdict."""
    res, case, out = _steps(config, steps, warmup, events=True)
    (pathlib.Path(root) / "timing").mkdir(parents=True, exist_ok=True)
    (pathlib.Path(root) / "timing" / "samples.json").write_text(
        json.dumps({"attention_ns": res.pop("attention_ns"), "call_ns": res.pop("call_ns")}) + "\n")
    res["correctness"] = dict(checker(case, out), checked=True) if checker else {"checked": False, "passed": False}
    res["passed"] = bool(res["correctness"]["passed"])
    return _write_result(pathlib.Path(root) / "timing", "timing", res)


def run_profiled(root, mode: str, config: str, steps: int, warmup: int) -> dict:
    """The same steps as a child process under rocprofv3 (the profiler preloads itself into the
    program after ``--``, so the child is python itself)."""
    phase_root = pathlib.Path(root) / mode
    phase_root.mkdir(parents=True, exist_ok=True)
    child = [sys.executable, "-m", "tpu_cake_amd.evidence", "_steps", "--config", config, "--steps", str(steps),
             "--warmup", str(warmup), "--out", str(phase_root / "steps.json")]
    env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
    env["PYTHONPATH"] = os.pathsep.join(filter(None, [str(PACKAGE.parent), str(PACKAGE.parents[1]),
                                                      env.get("PYTHONPATH", "")]))
    if mode == "trace":
        cmds = [["rocprofv3", "--kernel-trace", "--stats", "-d", str(phase_root / "kt"), "-o", "run",
                 "--output-format", "csv", "--"] + child]
    else:
        passes = [(c.lower(), [c]) for c in COUNTERS] + [("mfma", list(MFMA_COUNTERS))]
        cmds = [["rocprofv3", "--pmc", *cs, "-d", str(phase_root / d), "-o", "run", "--output-format", "csv",
                 "--"] + child for d, cs in passes]
    for cmd in cmds:
        subprocess.run(["timeout", "-s", "KILL", "120"] + cmd, check=True, env=env, stdout=subprocess.DEVNULL)
    steps_res = json.loads((phase_root / "steps.json").read_text())
    prof = inspect_profile(phase_root)
    assessment = assess_profile(prof, dispatches=steps,
                                counters=COUNTERS + MFMA_COUNTERS if mode == "counters" else ())
    body = {**steps_res, "profile": prof, "assessment": assessment, "passed": assessment["accepted"]}
    return _write_result(phase_root, mode, body)


# --------------------------------------------------------------------------- receipt
def _median(xs):
    s = sorted(xs)
    n = len(s)
    return (s[n // 2] + s[(n - 1) // 2]) / 2 if n else 0.0


def build_receipt(root) -> dict:
    """Accept three phase results as one run: same sources, same inputs, same configuration, every
    phase passed, every artifact hashed.  Writes ``receipt.json`` and returns it."""
    root = pathlib.Path(root)
    results = {m: json.loads((root / m / "result.json").read_text()) for m in PHASES}
    reasons = []
    for key in ("identity", "input_sha256", "config", "steps"):
        vals = {json.dumps(results[m].get(key), sort_keys=True) for m in PHASES}
        if len(vals) != 1:
            reasons.append(f"phases disagree on {key}")
    for m in PHASES:
        if not results[m].get("passed"):
            reasons.append(f"{m} phase did not pass")
    if not results["timing"]["correctness"].get("checked"):
        reasons.append("correctness was not checked")
    samples = json.loads((root / "timing" / "samples.json").read_text())
    trace_k = results["trace"]["profile"]["kernels"]
    cnt = results["counters"]["profile"]["counters"].get("rpa_attn_kernel", {})
    metrics = {
        "timing.attention_median_ns": _median(samples["attention_ns"]),
        "timing.call_median_ns": _median(samples["call_ns"]),
        "trace.attention_avg_ns": trace_k.get("rpa_attn_kernel", {}).get("avg_ns"),
        "trace.combine_avg_ns": trace_k.get("rpa_combine_kernel", {}).get("avg_ns"),
        "counters.attention_fetch_kib": cnt.get("FETCH_SIZE"),
        "counters.attention_write_kib": cnt.get("WRITE_SIZE"),
        "counters.attention_mfma_busy_cycles": cnt.get("SQ_VALU_MFMA_BUSY_CYCLES"),
        "counters.attention_gui_active_cycles": cnt.get("GRBM_GUI_ACTIVE"),
        "counters.attention_mfma_mops_bf16": cnt.get("SQ_INSTS_VALU_MFMA_MOPS_BF16"),
    }
    busy, active = metrics["counters.attention_mfma_busy_cycles"], metrics["counters.attention_gui_active_cycles"]
    if busy is not None and active:
        # GRBM_GUI_ACTIVE is summed over the 8 XCDs' instances, the busy cycles over 1024 SIMDs
        metrics["counters.attention_mfma_busy_fraction"] = round(busy / (active / 8 * 1024), 4)
    artifacts = []
    for m in PHASES:
        artifacts.append({"path": f"{m}/result.json", "sha256": sha256_file(root / m / "result.json"),
                          "role": f"{m}_result"})
        for a in results[m]["artifacts"]:
            artifacts.append({"path": f"{m}/{a['path']}", "sha256": a["sha256"], "role": a["role"]})
    receipt = {
        "status": "passed" if not reasons else "rejected",
        "reasons": reasons,
        "identity": results["timing"]["identity"],
        "config": results["timing"]["config"],
        "input_sha256": results["timing"]["input_sha256"],
        "correctness": results["timing"]["correctness"],
        "metrics": metrics,
        "assessments": {m: results[m]["assessment"] for m in ("trace", "counters")},
        "artifacts": artifacts,
    }
    (root / "receipt.json").write_text(json.dumps(receipt, indent=1, sort_keys=True) + "\n")
    return receipt


def validate_receipt(root) -> dict:
    """Re-check a receipt against the files: every artifact present with its hash, every phase
    result present, status consistent with the recorded reasons.  Raises ValueError."""
    root = pathlib.Path(root)
    receipt = json.loads((root / "receipt.json").read_text())
    for a in receipt["artifacts"]:
        p = root / a["path"]
        if not p.is_file():
            raise ValueError(f"RECEIPT_ARTIFACT_MISSING {a['path']}")
        if sha256_file(p) != a["sha256"]:
            raise ValueError(f"RECEIPT_ARTIFACT_CHANGED {a['path']}")
    roles = {a["role"] for a in receipt["artifacts"]}
    for m in PHASES:
        if f"{m}_result" not in roles:
            raise ValueError(f"RECEIPT_PHASE_MISSING {m}")
    if (receipt["status"] == "passed") != (not receipt["reasons"]):
        raise ValueError("RECEIPT_STATUS_INCONSISTENT")
    return receipt


def receipt_markdown(root, command: str) -> str:
    """A validated receipt as the markdown summary kept under ``profiles/``."""
    rec = validate_receipt(root)
    cfg = rec["config"]
    name = cfg.get("config", "?") if isinstance(cfg, dict) else str(cfg)
    corr = rec["correctness"]
    lines = [f"# Evidence receipt: {name.upper()} (timing, trace, counters)", "",
             "Command (repository root, MI355X box, `PYTHONPATH=tpu-cake_amd:.`):", "", "```", command,
             f"python -m tpu_cake_amd.evidence validate {root}", "```", "",
             f"Status: **{rec['status']}** (validated: every artifact re-hashed), kernel sources digest "
             f"{rec['identity'].get('kernel_source_digest', '?')}.", "", "| metric | value |", "|---|---|"]
    for k in sorted(rec["metrics"]):
        v = rec["metrics"][k]
        lines.append(f"| {k} | {v if v is not None else 'n/a'} |")
    lines += ["", f"Correctness (oracle `{corr.get('oracle', '?')}`): max-abs {corr.get('max_abs', float('nan')):.3e}, "
              f"rel-L2 {corr.get('rel_l2', float('nan')):.2e}, tolerance {corr.get('tolerance')}.", "",
              "Assessments: " + "; ".join(f"{m}: {'accepted' if a.get('accepted') else 'rejected'}"
                                          for m, a in sorted(rec["assessments"].items())), "",
              f"{len(rec['artifacts'])} artifacts (three result.json, timing samples, rocprofv3 CSVs) with sha256 "
              "in the receipt."]
    if rec["reasons"]:
        lines += ["", "Reasons: " + "; ".join(rec["reasons"])]
    return "\n".join(lines) + "\n"


# --------------------------------------------------------------------------- CLI
def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m tpu_cake_amd.evidence")
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("_steps")
    s.add_argument("--config", required=True)
    s.add_argument("--steps", type=int, required=True)
    s.add_argument("--warmup", type=int, required=True)
    s.add_argument("--out", required=True)
    i = sub.add_parser("inspect")
    i.add_argument("path")
    v = sub.add_parser("validate")
    v.add_argument("root")
    rm = sub.add_parser("receipt-md", help="write a validated receipt's markdown summary")
    rm.add_argument("root")
    rm.add_argument("--command", required=True, help="the command that produced the receipt")
    rm.add_argument("--write", required=True)
    pr = sub.add_parser("profile", help="run every rocprofv3 pass behind profiles/ (GPU box)")
    pr.add_argument("--raw", required=True)
    pr.add_argument("--configs", nargs="*", default=None)
    sm = sub.add_parser("summarize", help="write profiles/*.md and pmc_traffic.json from a profile run")
    sm.add_argument("--raw", required=True)
    sm.add_argument("--write", required=True)
    a = ap.parse_args(argv)
    if a.cmd in ("profile", "summarize"):
        from . import profiling

        if a.cmd == "profile":
            profiling.run_profiles(a.raw, tuple(a.configs) if a.configs else profiling.CONFIGS)
        else:
            profiling.summarize(a.raw, a.write, raw_label=a.raw)
        return 0
    if a.cmd == "_steps":
        res, _, _ = _steps(a.config, a.steps, a.warmup, events=False)
        pathlib.Path(a.out).write_text(json.dumps(res) + "\n")
        return 0
    if a.cmd == "receipt-md":
        pathlib.Path(a.write).write_text(receipt_markdown(a.root, a.command))
        return 0
    if a.cmd == "inspect":
        print(json.dumps(inspect_profile(a.path), indent=1, sort_keys=True))
        return 0
    rec = validate_receipt(a.root)
    print(f"RECEIPT_VALID status={rec['status']}")
    return 0


def run_all(root, config: str, steps: int, warmup: int, checker) -> dict:
    """Timing, trace and counters phases, then the receipt (validated)."""
    t0 = time.time()
    run_timing(root, config, steps, warmup, checker=checker)
    print(f"[evidence] timing done ({time.time() - t0:.0f}s)", flush=True)
    for mode in ("trace", "counters"):
        run_profiled(root, mode, config, steps, warmup)
        print(f"[evidence] {mode} done ({time.time() - t0:.0f}s)", flush=True)
    build_receipt(root)
    return validate_receipt(root)


if __name__ == "__main__":
    sys.exit(main())

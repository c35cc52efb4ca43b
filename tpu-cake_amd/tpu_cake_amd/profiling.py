"""The committed profiles: the rocprofv3 passes behind ``profiles/`` and the summaries made from them.

``run_profiles`` (on the GPU box) runs, for each configuration, ``bench.py`` under

* ``rocprofv3 --kernel-trace --stats`` (20 timed steps): per-kernel dispatch durations;
* ``rocprofv3 --pmc FETCH_SIZE`` and ``--pmc WRITE_SIZE`` (5 steps): HBM bytes per dispatch;
* ``rocprofv3 --pmc TCC_EA0_RDREQ_{128,64,32}B_sum TCC_EA0_WRREQ_64B_sum``: raw memory requests;
* ``rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_INSTS_VALU_MFMA_MOPS_BF16`` (C3, the
  configuration with MFMA-dense prefill rows, and C2): MFMA activity;

and a 1 GiB device copy under the FETCH_SIZE and WRITE_SIZE passes, whose readings calibrate
the two counters (bytes per KiB counted).  Every pass is its own process under
``timeout -s KILL``; raw output goes to ``RAW/<pass>_<config>/``.

``summarize`` (anywhere) turns ``RAW`` into ``profiles/rpa_attn_<config>.md``,
``profiles/rpa_fused_inkling.md`` and ``profiles/pmc_traffic.json`` (the per-dispatch HBM traffic
``bench.py`` reports as ``roofline.traffic``, keyed by the kernel-source digest).  The same raw
directory always gives the same files.

    PYTHONPATH=tpu-cake_amd python -m tpu_cake_amd.evidence profile --raw gpurun_out/prof   # GPU box
    PYTHONPATH=tpu-cake_amd python -m tpu_cake_amd.evidence summarize --raw gpurun_out/prof --write profiles
"""

from __future__ import annotations

import csv
import json
import os
import pathlib
import subprocess
import sys
from collections import defaultdict

PACKAGE = pathlib.Path(__file__).resolve().parent
ROOT = PACKAGE.parent.parent
CONFIGS = ("c1", "c2", "c3", "c4", "c5", "c2w", "c3f", "c5t", "c2d64", "c2d256", "inkling")
PASSES = {
    "fetch": ("FETCH_SIZE",),
    "write": ("WRITE_SIZE",),
    "tcc": ("TCC_EA0_RDREQ_128B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_32B_sum", "TCC_EA0_WRREQ_64B_sum"),
    "mfma": ("SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE", "SQ_INSTS_VALU_MFMA_MOPS_BF16"),
}
MFMA_CONFIGS = ("c2", "c3")
COPY_BYTES = 1 << 30
SIMDS = 256 * 4
# rocprofv3 sums a counter over its block's instances; GRBM has one per XCD, so the per-dispatch
# GRBM_GUI_ACTIVE is 8x the GPU's active cycles (its MfmaUtil takes the max over instances instead)
GRBM_INSTANCES = 8


def commands(raw: str, configs=CONFIGS) -> list[tuple[str, list[str]]]:
    """(name, argv) of every pass, in run order; argv runs from the repository root."""
    py = ["python3", "-u", "bench.py"]
    out = []
    for cfg in configs:
        out.append((f"prof_{cfg}", ["rocprofv3", "--kernel-trace", "--stats", "-d", f"{raw}/prof_{cfg}", "-o", cfg,
                                    "--output-format", "csv", "--", *py, "--config", cfg, "--steps", "20",
                                    "--warmup", "3", "--no-cpu-baseline"]))
        for name, counters in PASSES.items():
            if name == "mfma" and cfg not in MFMA_CONFIGS:
                continue
            if name == "tcc" and cfg == "inkling":
                continue
            out.append((f"{name}_{cfg}", ["rocprofv3", "--pmc", *counters, "-d", f"{raw}/{name}_{cfg}", "-o", cfg,
                                          "--output-format", "csv", "--", *py, "--config", cfg, "--steps", "5",
                                          "--warmup", "1", "--no-cpu-baseline"]))
    for name in ("fetch", "write"):
        out.append((f"{name}_copy", ["rocprofv3", "--pmc", *PASSES[name], "-d", f"{raw}/{name}_copy", "-o", "copy",
                                     "--output-format", "csv", "--", *py, "--copy-probe", str(COPY_BYTES)]))
    return out


def run_profiles(raw: str, configs=CONFIGS, limit_s: int = 120) -> None:
    """Run every pass (GPU box).  Stops at the first failing pass; the trace passes' bench lines go
    to ``RAW/prof_<config>.out``."""
    env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
    raw = str(pathlib.Path(raw).resolve())  # the passes run from the repository root
    pathlib.Path(raw).mkdir(parents=True, exist_ok=True)
    for name, argv in commands(raw, configs):
        argv = [sys.executable if a == "python3" else a for a in argv]
        print(f"[profile] {name}", flush=True)
        with open(pathlib.Path(raw) / f"{name}.out", "w") as fout:
            subprocess.run(["timeout", "-s", "KILL", str(limit_s), *argv], check=True, env=env, cwd=ROOT,
                           stdout=fout, stderr=subprocess.STDOUT)


# --------------------------------------------------------------------------- reading
def _short(name: str):
    from .evidence import _kernel_key

    return _kernel_key(name)


def _counters(d: pathlib.Path) -> dict:
    """kernel -> counter -> mean value per dispatch."""
    f = next(d.rglob("*counter_collection.csv"))
    per = defaultdict(lambda: defaultdict(float))
    disp = defaultdict(set)
    for r in csv.DictReader(open(f)):
        k = _short(r["Kernel_Name"])
        if k is None:
            continue
        per[k][r["Counter_Name"]] += float(r["Counter_Value"])
        disp[k].add(r["Dispatch_Id"])
    return {k: {c: v / len(disp[k]) for c, v in cs.items()} for k, cs in per.items()}


def _stats(d: pathlib.Path) -> dict:
    f = next(d.rglob("*kernel_stats.csv"))
    out = {}
    for r in csv.DictReader(open(f)):
        k = _short(r["Name"])
        if k and k.startswith("rpa"):
            out[k] = dict(calls=int(r["Calls"]), avg=float(r["AverageNs"]) / 1e3, min=float(r["MinNs"]) / 1e3,
                          max=float(r["MaxNs"]) / 1e3)
    return out


def _bench_line(path: pathlib.Path) -> dict:
    for line in reversed(path.read_text().splitlines()):
        if line.startswith("{"):
            return json.loads(line)
    raise ValueError(f"{path}: no bench line")


def _cmd_block(raw: str, cfg: str) -> str:
    rows = [" ".join(a) for n, a in commands(raw, (cfg,)) if not n.endswith("_copy")]
    rows += [" ".join(a) for n, a in commands(raw, ()) if n.endswith("_copy")]
    return "```\n" + "\n".join(rows) + "\n```"


def _trace_table(st: dict) -> str:
    rows = ["| kernel | calls | avg us | min us | max us |", "|---|---|---|---|---|"]
    for k, v in st.items():
        rows.append(f"| {k} | {v['calls']} | {v['avg']:.2f} | {v['min']:.2f} | {v['max']:.2f} |")
    return "\n".join(rows)


# --------------------------------------------------------------------------- summaries
def summarize(raw, out_dir, *, raw_label: str | None = None) -> dict:
    """Write the profile summaries and ``pmc_traffic.json`` from the raw pass outputs; returns the
    traffic table.  ``raw_label``: how the commands in the summaries name the raw directory."""
    from .evidence import kernel_source_digest
    from .workloads import CONFIG_DESCRIPTIONS, FUSED_DESCRIPTION, make_config_meta_for, make_fused_meta

    raw = pathlib.Path(raw)
    out_dir = pathlib.Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    label = raw_label or "gpurun_out/prof"
    digest = kernel_source_digest()
    copy_f = _counters(raw / "fetch_copy")["__amd_rocclr_copyBuffer"]["FETCH_SIZE"]
    copy_w = _counters(raw / "write_copy")["__amd_rocclr_copyBuffer"]["WRITE_SIZE"]
    kib = COPY_BYTES / 1024
    ff, wf = kib / copy_f, kib / copy_w
    traffic = {"source_sha256_16": digest, "fetch_factor": round(ff, 4), "write_factor": round(wf, 4),
               "configs": {}}
    configs = [c for c in CONFIGS if (raw / f"prof_{c}").exists()]
    for cfg in configs:
        if cfg == "inkling":
            continue
        meta, window = make_config_meta_for(cfg)
        work = meta.work(window)
        kv = work.kv_read_bytes + work.scale_bytes
        qo = work.q_bytes + work.o_bytes
        st = _stats(raw / f"prof_{cfg}")
        bj = _bench_line(raw / f"prof_{cfg}.out")
        fk = _counters(raw / f"fetch_{cfg}")["rpa_attn_kernel"]["FETCH_SIZE"]
        wk = _counters(raw / f"write_{cfg}")["rpa_attn_kernel"]["WRITE_SIZE"]
        tb = fk * 1024 * ff + wk * 1024 * wf
        avg = st["rpa_attn_kernel"]["avg"]
        ach = (kv + qo) / (avg * 1e-6) / 1e9
        entry = {"traffic_bytes": int(round(tb)), "fetch_kib": round(fk, 3), "write_kib": round(wk, 3),
                 "trace_avg_us": round(avg, 3), "algorithmic_bytes": kv + qo}
        tcc = ""
        if (raw / f"tcc_{cfg}").exists():
            t = _counters(raw / f"tcc_{cfg}")["rpa_attn_kernel"]
            r128, r64, r32 = (t.get(f"TCC_EA0_RDREQ_{b}B_sum", 0.0) for b in (128, 64, 32))
            tcc = (f"\n- raw TCC EA read requests: {(r128 * 128 + r64 * 64 + r32 * 32) / 1e6:.1f} MB "
                   f"(128B x {r128:.0f} + 64B x {r64:.0f} + 32B x {r32:.0f})")
        mfma = ""
        if (raw / f"mfma_{cfg}").exists():
            m = _counters(raw / f"mfma_{cfg}")["rpa_attn_kernel"]
            busy, active, mops = (m.get(c, 0.0) for c in ("SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE",
                                                           "SQ_INSTS_VALU_MFMA_MOPS_BF16"))
            util = busy / (active / GRBM_INSTANCES * SIMDS) if active else 0.0
            entry["mfma"] = {"busy_cycles": busy, "gui_active_cycles": active, "mfma_busy_fraction": round(util, 4),
                             "bf16_mfma_flops": mops * 512}
            mfma = (f"\n\n## MFMA activity of rpa_attn_kernel per dispatch\n\n"
                    f"- SQ_VALU_MFMA_BUSY_CYCLES {busy:.4g} (summed over SIMDs), GRBM_GUI_ACTIVE {active:.4g} "
                    f"(summed over the {GRBM_INSTANCES} XCDs): MFMA busy {util:.3f} of {SIMDS} SIMDs x active "
                    f"cycles (rocprofv3's MfmaUtil)\n"
                    f"- SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512 = {mops * 512 / 1e9:.1f} GFLOP issued on bf16 MFMA "
                    f"(algorithmic QK/PV of all rows: {work.flops / 1e9:.1f} GFLOP; prefill rows "
                    f"{work.prefill_flops / 1e9:.1f} GFLOP)")
        traffic["configs"][cfg] = entry
        extra = ""
        if work.prefill_flops:
            fl = work.prefill_flops
            extra = (f"\n- prefill FLOPs (causal) {fl / 1e9:.1f} GFLOP over the trace avg: "
                     f"{fl / (avg * 1e-6) / 1e12:.1f} TFLOP/s ({fl / (avg * 1e-6) / 2.5e15:.3f} of 2.5 PFLOP/s bf16; "
                     f"the decode rows share the launch)")
        desc = CONFIG_DESCRIPTIONS[meta.name] + (f"; sliding_window {window}" if window else "")
        md = f"""# rocprofv3 summary: {cfg} ({desc})

Kernel sources digest = {digest} (sha256[:16] of the sources without comments and blank space,
`tpu_cake_amd.evidence.kernel_source_digest`).  Made by `PYTHONPATH=tpu-cake_amd python -m tpu_cake_amd.evidence profile --raw {label}`
on the MI355X box (the passes below, from the repository root) and
`PYTHONPATH=tpu-cake_amd python -m tpu_cake_amd.evidence summarize --raw {label} --write profiles`.

{_cmd_block(label, cfg)}

## Kernel trace (--stats)

{_trace_table(st)}

bench.py in the same traced run: attention kernel (HIP events) avg {bj['attn_kernel_ms']['avg'] * 1e3:.2f} us,
step {bj['ms_per_step'] * 1e3:.2f} us.

## HBM traffic of rpa_attn_kernel per dispatch

- FETCH_SIZE {fk:.0f} KiB x {ff:.3f} (copy calibration) = {fk * 1024 * ff / 1e6:.1f} MB
- WRITE_SIZE {wk:.0f} KiB x {wf:.3f} = {wk * 1024 * wf / 1e6:.2f} MB{tcc}
- algorithmic bytes (tpu_cake_amd.cost_model.rpa_work): KV {kv / 1e6:.1f} MB + Q/O {qo / 1e6:.2f} MB;
  traffic / algorithmic = {tb / (kv + qo):.3f}
- achieved (algorithmic KV+Q+O over the trace avg {avg:.2f} us): {ach:.0f} GB/s ({ach / 8000:.3f} of 8 TB/s){extra}{mfma}

Copy calibration: a 1 GiB device copy reads FETCH_SIZE = {copy_f:.0f} KiB (factor {ff:.3f}) and writes
WRITE_SIZE = {copy_w:.0f} KiB (factor {wf:.3f}).
"""
        (out_dir / f"rpa_attn_{cfg}.md").write_text(md)
    if "inkling" in configs:
        fm = make_fused_meta()
        st = _stats(raw / "prof_inkling")
        bj = _bench_line(raw / "prof_inkling.out")
        cf, cw = _counters(raw / "fetch_inkling"), _counters(raw / "write_inkling")
        lines, tot = [], 0.0
        for k in ("rpa_fused_prep_kernel", "rpa_attn_kernel", "rpa_combine_kernel"):
            if k not in cf or k not in cw:  # the one-launch form of the step has no prep launch
                continue
            b = cf[k]["FETCH_SIZE"] * 1024 * ff + cw[k]["WRITE_SIZE"] * 1024 * wf
            tot += b
            lines.append(f"- {k}: FETCH_SIZE {cf[k]['FETCH_SIZE']:.0f} KiB x {ff:.3f}, WRITE_SIZE "
                         f"{cw[k]['WRITE_SIZE']:.0f} KiB x {wf:.3f} = {b / 1e6:.2f} MB")
        ksum = sum(v["avg"] for v in st.values())
        moved = fm["moved_bytes"]
        ach = moved / (ksum * 1e-6) / 1e9
        traffic["configs"]["inkling"] = {"traffic_bytes": int(round(tot)), "basis": "whole step",
                                         "kernels_avg_us": {k: round(v["avg"], 3) for k, v in st.items()}}
        md = f"""# rocprofv3 summary: inkling ({FUSED_DESCRIPTION})

Kernel sources digest = {digest}.  Made by `PYTHONPATH=tpu-cake_amd python -m tpu_cake_amd.evidence profile --raw {label}` and
`PYTHONPATH=tpu-cake_amd python -m tpu_cake_amd.evidence summarize --raw {label} --write profiles`:

{_cmd_block(label, 'inkling')}

## Kernel trace (--stats)

{_trace_table(st)}

bench.py in the same traced run: step {bj['ms_per_step'] * 1e3:.2f} us (HIP events around the whole call); the
kernels sum to {ksum:.2f} us.

## HBM traffic of one step per dispatch

{chr(10).join(lines)}
- algorithmic bytes per step (KV + Q + O + new K/V rows) {moved / 1e6:.1f} MB; traffic / algorithmic = {tot / moved:.3f}
- achieved over the kernels ({ksum:.2f} us): {ach:.0f} GB/s ({ach / 8000:.3f} of 8 TB/s)
"""
        (out_dir / "rpa_fused_inkling.md").write_text(md)
    (out_dir / "pmc_traffic.json").write_text(json.dumps(traffic, indent=1, sort_keys=True) + "\n")
    return traffic

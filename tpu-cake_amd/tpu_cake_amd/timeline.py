"""Per-workgroup timeline of ``rpa_attn_kernel``: where a launch's time goes, workgroup by workgroup.

    PYTHONPATH=tpu-cake_amd python -m tpu_cake_amd.timeline --config c3 [--runs 8] [--write FILE] [--raw FILE]

Runs the configuration's operator call (the call ``bench.py --config`` times: same case, knobs from
the tuned table, KV pools rotated) through ``librpa_timeline.so`` -- the library built from the same
sources with ``-DRPA_TIMELINE`` (``tpu_cake_amd.build``) -- and reads the attention kernel's
timeline of the last run with ``rpa_timeline_read``: per workgroup, stamps of the 100 MHz constant
clock at its phases, its role, its work, per-tile phase sums of its prefill tiles, and the XCD and
CU it ran on.  The printed summary (markdown) gives the launch's span against the HIP-event
duration of the same launch (which checks the clock rate), the start spread, the stream-K role's
start-up and end spread, the prefill tiles' step rate and per-tile overheads, and the placement
facts the schedule relies on (workgroup b on XCD b mod 8; in the co-resident layout b and
b + grid/2 on one CU).  The instrumented kernel is not the product kernel: its stamps add a few
instructions per phase and per tile, so compare its HIP-event duration with the product's.
"""

from __future__ import annotations

import argparse
import ctypes
import math
import os
import pathlib
import statistics
import sys

PACKAGE = pathlib.Path(__file__).resolve().parent
TIMELINE_LIB = PACKAGE / "librpa_timeline.so"
FIELDS = ("start", "sched", "first", "dec", "tiles0", "ranked", "end", "role", "units", "ntiles", "nsteps",
          "queue", "setup", "loop", "write", "where")
NF = len(FIELDS)
TICK_US = 0.01  # s_memrealtime: 100 MHz


def _q(xs, f):
    xs = sorted(xs)
    if not xs:
        return float("nan")
    return xs[min(len(xs) - 1, int(round(f * (len(xs) - 1))))]


def summarize(rows: list[dict], grid: int, waves: int, kernel_us: float) -> list[str]:
    """Markdown lines for one launch's rows (workgroup b = rows[b])."""
    t0 = min(r["start"] for r in rows)
    us = lambda t: (t - t0) * TICK_US  # noqa: E731
    span = (max(r["end"] for r in rows) - t0) * TICK_US
    out = [f"- launch: {grid} workgroups x {waves} waves; HIP-event duration {kernel_us:.2f} us; timeline span "
           f"(first start to last exit) {span:.2f} us (the two agree when the clock runs at 100 MHz)",
           f"- workgroup starts: median {statistics.median(us(r['start']) for r in rows):.2f} us, "
           f"max {max(us(r['start']) for r in rows):.2f} us after the first"]
    sk = [r for r in rows if r["role"] & 2]
    if sk:
        first = [us(r["first"]) for r in sk]
        dec = [us(r["dec"]) for r in sk]
        units = [r["units"] for r in sk]
        out += [f"- stream-K workgroups with a range: {len(sk)}; units per range median {statistics.median(units):.0f} "
                f"(min {min(units)}, max {max(units)})",
                f"  - work split known (all workgroups): median {statistics.median(us(r['sched']) for r in rows):.2f} us",
                f"  - first unit's loads issued: median {statistics.median(first):.2f} us, p90 {_q(first, .9):.2f}",
                f"  - range done: median {statistics.median(dec):.2f} us, p10 {_q(dec, .1):.2f}, "
                f"p90 {_q(dec, .9):.2f}, max {max(dec):.2f}"]
    tiled = [r for r in rows if r["ntiles"] > 0]
    if tiled:
        steps = sum(r["nsteps"] for r in tiled)
        tiles = sum(r["ntiles"] for r in tiled)
        loop = sum(r["loop"] for r in tiled) * TICK_US
        pf = [r for r in tiled if r["role"] & 1]
        joined = [r for r in tiled if r["role"] & 4]
        out += [f"- prefill tiles: {tiles} tiles (or tile parts), {steps} chunk steps of 32 keys x 128 rows, "
                f"taken by {len(pf)} prefill-first and {len(joined)} joining workgroups",
                f"  - step loop: {loop / steps:.3f} us per step over all workgroups"]
        for label, grp in (("prefill-first", pf), ("joining", joined)):
            if not grp:
                continue
            st = sum(r["nsteps"] for r in grp)
            nt = sum(r["ntiles"] for r in grp)
            out.append(f"  - {label}: {sum(r['loop'] for r in grp) * TICK_US / max(st, 1):.3f} us per step; per tile: "
                       f"set-up {sum(r['setup'] for r in grp) * TICK_US / nt:.2f} us, queue fetch "
                       f"{sum(r['queue'] for r in grp) * TICK_US / nt:.2f} us, row writes "
                       f"{sum(r['write'] for r in grp) * TICK_US / nt:.2f} us; tile order ready "
                       f"{statistics.median(us(r['ranked']) - us(r['tiles0']) for r in grp):.2f} us after the role "
                       f"starts (median); steps per workgroup max {max(r['nsteps'] for r in grp)}")
        if pf:
            out.append(f"  - prefill-first workgroups end: median {statistics.median(us(r['end']) for r in pf):.2f} us, "
                       f"max {max(us(r['end']) for r in pf):.2f}")
    ends = [us(r["end"]) for r in rows]
    out.append(f"- workgroup exits: p10 {_q(ends, .1):.2f} us, median {statistics.median(ends):.2f}, "
               f"p90 {_q(ends, .9):.2f}, max {max(ends):.2f}")
    xcc = [(r["where"] >> 32) & 0xF for r in rows]
    out.append(f"- placement: workgroup b on XCD b mod 8 for {sum(x == b % 8 for b, x in enumerate(xcc))} of {len(rows)} "
               f"workgroups")
    if grid % 2 == 0:
        half = grid // 2
        cu = [((r["where"] >> 32) & 0xF, (r["where"] >> 8) & 0xFF) for r in rows]
        same = sum(cu[b] == cu[b + half] for b in range(half))
        out.append(f"  - workgroups b and b + {half} on one CU (XCC_ID and HW_ID's CU, shader array and engine "
                   f"fields) for {same} of {half} pairs; distinct CUs used: {len(set(cu))}")
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--config", default="c3", choices=["c1", "c2", "c3", "c4", "c5", "c2w", "c3f", "c5t", "c2d64", "c2d256"])
    ap.add_argument("--seed", type=int, default=None)
    ap.add_argument("--runs", type=int, default=8, help="calls before the one whose timeline is read")
    ap.add_argument("--write", default=None, help="also write the summary to this file")
    ap.add_argument("--raw", default=None, help="also write the rows (one JSON object per workgroup) to this file")
    args = ap.parse_args(argv)
    if not TIMELINE_LIB.exists():
        print(f"{TIMELINE_LIB} missing: build it with `python -m tpu_cake_amd.build`", file=sys.stderr)
        return 2
    os.environ["RPA_LIB"] = str(TIMELINE_LIB)  # before the first load of the library

    import torch

    from . import _lib, ops
    from .timing import KernelEvent
    from .workloads import CONFIG_DESCRIPTIONS, WINDOWED_CONFIGS, make_config

    if not torch.cuda.is_available():
        print("timeline: no GPU visible", file=sys.stderr)
        return 2
    lib = _lib.load()
    base, window = WINDOWED_CONFIGS.get(args.config, (args.config, None))
    case = make_config(base, seed=args.seed)
    dev = torch.device("cuda", 0)
    d = ops.case_to_device(case, dev)
    kv_scales = d.pop("kv_scales", None)
    pool_bytes = d["kv_pages"].numel() * d["kv_pages"].element_size()
    copies = max(2, math.ceil(2.0e9 / pool_bytes))
    pools = [d["kv_pages"]] + [d["kv_pages"].clone() for _ in range(copies - 1)]
    out = torch.empty_like(d["q"])
    ev = (KernelEvent(), KernelEvent())
    for i in range(args.runs + 1):
        ops.ragged_paged_attention(d["q"], pools[i % copies], d["kv_lens"], d["page_indices"], d["cu_q_lens"],
                                   d["num_seqs"], sm_scale=case.sm_scale, kv_scales=kv_scales, out=out,
                                   sliding_window=window, kernel_events=ev)
    torch.cuda.synchronize()
    kernel_us = ev[0].elapsed_time(ev[1]) * 1e3
    grid, waves = ops.attention_grid(case)
    buf = (ctypes.c_int64 * (grid * NF))()
    rc = lib.rpa_timeline_read(buf, grid, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    if rc != 0:
        print(f"rpa_timeline_read failed ({rc}): {lib.rpa_last_error().decode()}", file=sys.stderr)
        return 1
    rows = [dict(zip(FIELDS, buf[b * NF:(b + 1) * NF])) for b in range(grid)]
    if any(r["start"] == 0 or r["end"] < r["start"] for r in rows):
        print("timeline: some workgroup rows were not written by the last launch", file=sys.stderr)
        return 1
    desc = CONFIG_DESCRIPTIONS[base] + (f"; sliding_window {window}" if window else "")
    lines = [f"# rpa_attn_kernel timeline, {args.config}", "",
             f"Workload: {args.config}: {desc}.", "",
             "Command: `PYTHONPATH=tpu-cake_amd python -m tpu_cake_amd.timeline --config "
             f"{args.config}" + (f" --seed {args.seed}" if args.seed is not None else "") + "` (the "
             "`-DRPA_TIMELINE` build of the same sources; the last of "
             f"{args.runs + 1} calls, KV pools rotated over {copies} copies; times from the first workgroup's "
             "start).", ""]
    lines += summarize(rows, grid, waves, kernel_us)
    text = "\n".join(lines) + "\n"
    print(text, flush=True)
    if args.write:
        pathlib.Path(args.write).write_text(text)
    if args.raw:
        import json

        pathlib.Path(args.raw).write_text(json.dumps({"grid": grid, "waves": waves, "kernel_us": kernel_us,
                                                      "fields": FIELDS, "rows": [list(buf[b * NF:(b + 1) * NF])
                                                                                 for b in range(grid)]}))
    return 0


if __name__ == "__main__":
    sys.exit(main())

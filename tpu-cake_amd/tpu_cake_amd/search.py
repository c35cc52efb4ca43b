"""Latin-square search over the RPA kernel's schedule knobs, with the reference's protocol.

The reference searches Pallas block sizes (``src/tpu_cake/rpa_search.py:564-661``).  The stream-K
kernel here has no block sizes -- its schedule balances work by itself -- so the searched
parameters are the per-call knobs of ``rpa_options_t`` (``waves_per_cu``, ``prefill_tiles``,
``prefill_cost``).  Everything else follows the reference:

* **contract** (``RpaSearchContract``, :71-110): configuration, seed, warmup / measured calls,
  rounds (whole forward + reversed Latin squares), confirmation rounds (even), bootstrap samples,
  the minimum practical improvement (1%), the candidates (unique names and knob sets) and the
  baseline.  It is written to ``contract.json`` and a resumed search must present the same one
  (``RPA_SEARCH_CONTRACT_CHANGED``, :586-591).
* **runs**: one per (round, position), ``round-RR/PP-name``, each a fresh child process under
  ``rocprofv3 --kernel-trace`` running warmup + measured calls of the configuration with the
  candidate's knobs.  The objective is the DEVICE time per call taken from that trace -- the
  dispatch durations of each measured call's kernels -- as the reference takes its
  from the XProf device events (``_device_timing``, :228-265); ``device_timing.json`` must replay
  from the trace (``RPA_SEARCH_DEVICE_TIMING_REPLAY_MISMATCH``).
* **correctness gate**: before the squares each candidate runs once (``gate/NN-name``, which keeps
  its output) and the caller's checker judges that output (the reference's run gate, :610-631); a
  failing candidate is dropped and never timed.  Every later run of a candidate must reproduce the
  gated output bits (their sha256; the reference pins the output hash per candidate, :418-429).
* **statistics** (:266-327): per round, the candidate's run median is paired with the baseline's run
  median of the same round, improvement = (baseline - candidate) / baseline; a bootstrap of the
  median of those paired improvements gives a 95% interval, and a candidate is promotable when the
  interval's low end exceeds the minimum practical improvement.  The provisional winner is the
  promotable candidate with the largest median improvement.
* **confirmation** (:330-354): fresh rounds alternating (baseline, winner) and (winner, baseline);
  the winner is confirmed when their paired interval's low end exceeds the threshold.
* **resume** (:574-621): a run with ``result.json`` is re-validated and reused; a run directory
  without one is moved to ``incomplete/<round>/<run>-attempt-NN`` with a ``failure.json``
  (``_archive_incomplete_run``, :544-561), and run again.

``--promote`` writes a confirmed winner into the tuned table (``tpu_cake_amd.tuned``) under the
configuration's shape key.

    python -m tpu_cake_amd.search --config c3 --root OUT --checker tests/evidence_run.py \\
        --candidate base: --candidate pf35:prefill_cost=0.35 --candidate pf60:prefill_cost=0.6
"""

from __future__ import annotations

import argparse
import csv
import dataclasses
import hashlib
import json
import os
import pathlib
import statistics as pystats
import subprocess
import sys

import numpy as np

from . import tuned

KNOBS = tuned.KNOBS


# --------------------------------------------------------------------------- contract
@dataclasses.dataclass(frozen=True)
class SearchContract:
    config: str
    baseline: str
    candidates: tuple  # ((name, {knob: value}), ...) in declaration order
    rounds: int
    confirmation_rounds: int = 2
    seed: int | None = None
    warmup: int = 5
    steps: int = 50
    bootstrap_samples: int = 10_000
    minimum_practical_improvement: float = 0.01

    def __post_init__(self):
        names = [n for n, _ in self.candidates]
        knob_sets = [json.dumps(tuned.validate_entry(k), sort_keys=True) for _, k in self.candidates]
        if len(names) < 2:
            raise ValueError("RPA search needs at least two candidates")
        if len(names) != len(set(names)) or len(knob_sets) != len(set(knob_sets)):
            raise ValueError("RPA search candidates need unique names and knob sets")
        if self.baseline not in names:
            raise ValueError("RPA search baseline must name one candidate")
        if self.rounds <= 0 or self.rounds % (2 * len(names)):
            raise ValueError("RPA search rounds must complete forward and reverse Latin squares")
        if self.confirmation_rounds < 0 or self.confirmation_rounds % 2:
            raise ValueError("RPA confirmation rounds must balance both run orders")
        if self.bootstrap_samples < 1000:
            raise ValueError("RPA search needs at least 1000 bootstrap samples")
        if not 0.0 < self.minimum_practical_improvement < 1.0:
            raise ValueError("minimum_practical_improvement must lie in (0, 1)")
        if self.steps < 1 or self.warmup < 0:
            raise ValueError("RPA search needs at least one measured call")

    @property
    def names(self) -> tuple:
        return tuple(n for n, _ in self.candidates)

    def knobs(self, name: str) -> dict:
        return tuned.validate_entry(dict(self.candidates)[name])

    def to_json(self) -> dict:
        d = dataclasses.asdict(self)
        d["candidates"] = [[n, tuned.validate_entry(k)] for n, k in self.candidates]
        return d

    @property
    def search_id(self) -> str:
        text = json.dumps(self.to_json(), sort_keys=True, separators=(",", ":"))
        return hashlib.sha256(text.encode()).hexdigest()


def execution_orders(names, rounds: int):
    """Round r runs the candidates rotated by r % n, in forward order in even squares and reversed
    order in odd squares (square = r // n) -- ``_execution_orders``, rpa_search.py:201-210."""
    names = tuple(names)
    n = len(names)
    if rounds % (2 * n):
        raise ValueError("search rounds must complete forward and reverse Latin squares")
    orders = []
    for r in range(rounds):
        basis = names if (r // n) % 2 == 0 else tuple(reversed(names))
        k = r % n
        orders.append(basis[k:] + basis[:k])
    return tuple(orders)


# --------------------------------------------------------------------------- statistics
@dataclasses.dataclass(frozen=True)
class DeviceTiming:
    """Per-call device time of one run's measured calls (ns) and its median / p90."""
    durations_ns: tuple
    median_ns: float
    p90_ns: float

    @staticmethod
    def of(durations) -> "DeviceTiming":
        d = tuple(float(x) for x in durations)
        if not d or any(x <= 0 for x in d):
            raise ValueError("device timing needs positive durations")
        return DeviceTiming(d, float(pystats.median(d)), float(_percentile(d, 0.9)))

    def to_json(self) -> dict:
        return {"durations_ns": list(self.durations_ns), "median_ns": self.median_ns, "p90_ns": self.p90_ns}


def _percentile(values, fraction: float):
    s = sorted(values)
    return s[min(len(s) - 1, round((len(s) - 1) * fraction))]


def improvement_interval(paired, *, samples: int, seed: int) -> tuple:
    """95% bootstrap interval of the median of the paired improvements (rpa_search.py:266-279)."""
    gen = np.random.default_rng(seed)
    values = np.asarray(paired, dtype=np.float64)
    est = np.empty(samples, dtype=np.float64)
    for i in range(samples):
        est[i] = np.median(gen.choice(values, len(values), replace=True))
    lo, hi = np.quantile(est, (0.025, 0.975))
    return float(lo), float(hi)


def paired_improvements(baseline_runs, candidate_runs) -> list:
    if len(baseline_runs) != len(candidate_runs):
        raise ValueError("paired statistics need one baseline run per candidate run")
    return [(b.median_ns - c.median_ns) / b.median_ns for b, c in zip(baseline_runs, candidate_runs)]


def statistics(contract: SearchContract, results: dict) -> dict:
    """results: name -> [DeviceTiming per round].  Per candidate: run and sample counts, median of
    the run medians, p90 of the run medians, median absolute deviation and coefficient of
    variation of the run medians, the median paired improvement over the baseline with its
    bootstrap interval, and whether it is promotable (rpa_search.py:282-327)."""
    base = results[contract.baseline]
    seed0 = int(contract.search_id[:16], 16)
    out = {}
    for idx, name in enumerate(contract.names):
        if name not in results:
            continue
        runs = results[name]
        meds = [r.median_ns for r in runs]
        paired = paired_improvements(base, runs)
        lo, hi = improvement_interval(paired, samples=contract.bootstrap_samples, seed=seed0 ^ idx)
        med = float(pystats.median(meds))
        mean = pystats.mean(meds)
        out[name] = {
            "runs": len(runs), "samples": sum(len(r.durations_ns) for r in runs), "median_ns": med,
            "p90_run_median_ns": float(_percentile(meds, 0.9)),
            "mad_ns": float(pystats.median(abs(m - med) for m in meds)),
            "cv": (pystats.pstdev(meds) / mean) if len(meds) > 1 and mean else 0.0,
            "improvement": float(pystats.median(paired)), "improvement_ci95": [lo, hi],
            "promotable": name != contract.baseline and lo > contract.minimum_practical_improvement,
        }
    return out


def confirmation_statistics(contract: SearchContract, candidate: str, orders, baseline_runs,
                            candidate_runs) -> dict:
    """Confirmation rounds: paired improvements of the winner over the baseline, bootstrap interval,
    confirmed when its low end exceeds the minimum practical improvement (rpa_search.py:330-354)."""
    paired = paired_improvements(baseline_runs, candidate_runs)
    lo, hi = improvement_interval(paired, samples=contract.bootstrap_samples,
                                  seed=int(contract.search_id[16:32], 16))
    return {"baseline": contract.baseline, "candidate": candidate, "runs": len(paired),
            "orders": [list(o) for o in orders], "improvement": float(pystats.median(paired)),
            "improvement_ci95": [lo, hi], "confirmed": lo > contract.minimum_practical_improvement}


# --------------------------------------------------------------------------- run artifacts
CALL_KERNELS = ("rpa_attn_kernel", "rpa_prefill_kernel", "rpa_combine_kernel")


def device_timing(run_root: pathlib.Path, steps: int) -> DeviceTiming:
    """Device time per measured call from the run's rocprofv3 kernel trace: a call is an attention
    dispatch and the call's other dispatches up to the next one (the prefill kernel and its
    combine, when the call uses them); the last ``steps`` calls are the measured ones, and a call's
    time is the sum of its dispatch durations."""
    traces = sorted(pathlib.Path(run_root).rglob("*kernel_trace.csv"))
    if len(traces) != 1:
        raise ValueError(f"RPA_SEARCH_TRACE_COUNT_MISMATCH path={run_root} traces={len(traces)}")
    rows = []
    for r in csv.DictReader(open(traces[0])):
        name = r["Kernel_Name"]
        kind = next((k for k in CALL_KERNELS if k in name), None)
        if kind is not None:
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), kind))
    rows.sort()
    calls: list[list] = []
    for start, end, kind in rows:
        if kind == CALL_KERNELS[0]:
            calls.append([])
        elif not calls:
            raise ValueError(f"RPA_SEARCH_DISPATCH_PROTOCOL_MISMATCH path={run_root} {kind} before any attention")
        calls[-1].append((kind, end - start))
    shapes = {tuple(k for k, _ in c) for c in calls}
    if len(calls) < steps or len(shapes) != 1:
        raise ValueError(f"RPA_SEARCH_DISPATCH_PROTOCOL_MISMATCH path={run_root} calls={len(calls)} "
                         f"expected >= {steps} of one dispatch sequence, got {sorted(shapes)}")
    return DeviceTiming.of([sum(d for _, d in c) for c in calls[-steps:]])


def _sha256(path: pathlib.Path) -> str:
    return hashlib.sha256(pathlib.Path(path).read_bytes()).hexdigest()


def archive_incomplete_run(search_root: pathlib.Path, run_root: pathlib.Path, reason: str) -> pathlib.Path:
    """Move an unfinished run aside as ``incomplete/<parent>/<name>-attempt-NN`` with a
    ``failure.json`` giving the reason (rpa_search.py:544-561)."""
    (run_root / "failure.json").write_text(json.dumps({"reason": reason}, sort_keys=True, indent=2) + "\n")
    rel = run_root.relative_to(search_root)
    parent = search_root / "incomplete" / rel.parent
    parent.mkdir(parents=True, exist_ok=True)
    attempt = 0
    while True:
        dst = parent / f"{rel.name}-attempt-{attempt:02d}"
        if not dst.exists():
            run_root.rename(dst)
            return dst
        attempt += 1


def incomplete_attempts(search_root: pathlib.Path) -> list:
    """Archived attempts with a manifest hash over (path, size, sha256) of their files."""
    root = pathlib.Path(search_root) / "incomplete"
    if not root.exists():
        return []
    out = []
    for att in sorted(p for p in root.rglob("*-attempt-*") if p.is_dir()):
        files = sorted(p for p in att.rglob("*") if p.is_file())
        manifest = [{"path": p.relative_to(att).as_posix(), "size_bytes": p.stat().st_size, "sha256": _sha256(p)}
                    for p in files]
        enc = json.dumps(manifest, sort_keys=True, separators=(",", ":")).encode()
        out.append({"path": att.relative_to(search_root).as_posix(), "file_count": len(files),
                    "total_size_bytes": sum(m["size_bytes"] for m in manifest),
                    "manifest_sha256": hashlib.sha256(enc).hexdigest()})
    return out


# --------------------------------------------------------------------------- runners
class TraceRunner:
    """Runs one search run as a child process under ``rocprofv3 --kernel-trace``: the child builds
    the configuration, makes warmup + measured calls with the candidate's knobs and saves its
    output; the profiler writes the kernel trace the objective is read from."""

    def __init__(self, rocprof: str = "rocprofv3", timeout_s: int = 300):
        self.rocprof, self.timeout_s = rocprof, timeout_s

    def run(self, run_root: pathlib.Path, contract: SearchContract, knobs: dict, save_output: bool = False) -> None:
        run_root.mkdir(parents=True, exist_ok=True)
        pkg = pathlib.Path(__file__).resolve().parent
        child = [sys.executable, "-m", "tpu_cake_amd.search", "_run", "--config", contract.config,
                 "--knobs", json.dumps(knobs, sort_keys=True), "--steps", str(contract.steps),
                 "--warmup", str(contract.warmup), "--out", str(run_root)]
        if save_output:
            child.append("--save-output")
        if contract.seed is not None:
            child += ["--seed", str(contract.seed)]
        env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
        env["PYTHONPATH"] = os.pathsep.join(filter(None, [str(pkg.parent), str(pkg.parents[1]),
                                                          env.get("PYTHONPATH", "")]))
        cmd = ["timeout", "-k", "10", str(self.timeout_s), self.rocprof, "--kernel-trace", "-d",
               str(run_root / "trace"), "-o", "run", "--output-format", "csv", "--"] + child
        subprocess.run(cmd, check=True, env=env, stdout=subprocess.DEVNULL)


def _child_run(config: str, knobs: dict, steps: int, warmup: int, out: pathlib.Path, seed,
               save_output: bool) -> None:
    """The child process of a run: the steps, their identity, the output's sha256 and (gate runs) the
    output's bits."""
    from . import evidence

    res, case, o = evidence._steps(config, steps, warmup, events=False, seed=seed, knobs=knobs)
    if save_output:
        import torch

        np.save(out / "output.npy", o.view(torch.int16).cpu().numpy().view(np.uint16))
    res["identity"] = evidence.source_identity()
    (out / "steps.json").write_text(json.dumps(res, sort_keys=True) + "\n")


def load_output(run_root: pathlib.Path) -> np.ndarray:
    """A run's saved output as float32 (from its bf16 bits)."""
    bits = np.load(pathlib.Path(run_root) / "output.npy", allow_pickle=False)
    return (bits.astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------------------- the search
def refuse_noop_candidates(contract: SearchContract, case, grid_of) -> None:
    """Refuse a candidate that differs from the baseline only in ``waves_per_cu`` and resolves to
    the baseline's launch (``grid_of(case, knobs) -> (workgroups, waves per workgroup)``, the
    library's ``rpa_attention_grid``): timing it against the baseline would compare identical
    launches."""
    base = contract.knobs(contract.baseline)
    base_grid = None
    for name in contract.names:
        k = contract.knobs(name)
        if name == contract.baseline or {**k, "waves_per_cu": base["waves_per_cu"]} != base:
            continue
        base_grid = base_grid or grid_of(case, base)
        g = grid_of(case, k)
        if g == base_grid:
            raise ValueError(f"RPA_SEARCH_NOOP_CANDIDATE candidate={name}: waves_per_cu={k['waves_per_cu']} "
                             f"resolves to the baseline's launch ({g[0]} workgroups of {g[1]} waves)")


def _device_grid(case, knobs) -> tuple:
    from . import ops

    return ops.attention_grid(case, knobs, cus=0)


def run_search(root, contract: SearchContract, *, runner, checker, case=None, keep_outputs: bool = False,
               grid_of=_device_grid) -> dict:
    """Run (or resume) a search; ``checker(case, output_f32) -> {"passed": bool, ...}`` is the
    correctness gate (``case`` defaults to the configuration's workload, built once here).  A gate
    run's output is deleted once its verdict is written (its sha256 stays in ``steps.json``) unless
    ``keep_outputs``.  Candidates that resolve to the baseline's launch are refused first
    (``refuse_noop_candidates``; ``grid_of`` None skips that).  Writes ``result.json`` under
    ``root`` and returns it."""
    root = pathlib.Path(root).resolve()
    root.mkdir(parents=True, exist_ok=True)
    cpath = root / "contract.json"
    ctext = json.dumps(contract.to_json(), indent=1, sort_keys=True) + "\n"
    if cpath.exists():
        if cpath.read_text() != ctext:
            raise ValueError("RPA_SEARCH_CONTRACT_CHANGED")
    else:
        cpath.write_text(ctext)

    identities: dict = {}  # candidate -> (output sha256, input sha256)
    shared: dict = {}      # identity every run must share (sources, library, inputs)

    def validate_run(run_root: pathlib.Path, name: str) -> DeviceTiming:
        steps = json.loads((run_root / "steps.json").read_text())
        ident = {"identity": steps["identity"], "input_sha256": steps["input_sha256"], "config": steps["config"]}
        if not shared:
            shared.update(ident)
        elif ident != shared:
            raise ValueError(f"RPA_SEARCH_EXECUTION_IDENTITY_MISMATCH run={run_root.relative_to(root)}")
        if steps["knobs"] != contract.knobs(name):
            raise ValueError(f"RPA_SEARCH_KNOB_MISMATCH run={run_root.relative_to(root)}")
        out_sha = steps["output_sha256"]
        if name in identities and identities[name] != out_sha:
            raise ValueError(f"RPA_SEARCH_CANDIDATE_OUTPUT_MISMATCH candidate={name}")
        identities.setdefault(name, out_sha)
        timing = device_timing(run_root, contract.steps)
        tpath = run_root / "device_timing.json"
        if not tpath.exists():
            tpath.write_text(json.dumps(timing.to_json(), indent=1) + "\n")
        saved = json.loads(tpath.read_text())
        if saved != json.loads(json.dumps(timing.to_json())):
            raise ValueError(f"RPA_SEARCH_DEVICE_TIMING_REPLAY_MISMATCH candidate={name}")
        return timing

    def ensure_run(rel: str, name: str, save_output: bool = False) -> DeviceTiming:
        run_root = root / rel
        if (run_root / "result.json").exists():
            return validate_run(run_root, name)
        if run_root.exists():
            archive_incomplete_run(root, run_root, "incomplete run found during resume")
        try:
            runner.run(run_root, contract, contract.knobs(name), save_output=save_output)
            timing = validate_run(run_root, name)
        except Exception as err:
            if run_root.exists():
                archive_incomplete_run(root, run_root, f"{type(err).__name__}: {err}")
            raise
        (run_root / "result.json").write_text(json.dumps(
            {"candidate": name, "knobs": contract.knobs(name), "output_sha256": identities[name],
             "device_median_ns": timing.median_ns}, indent=1, sort_keys=True) + "\n")
        return timing

    # the correctness gate: one checked run per candidate; failures are dropped
    gate = {}
    if case is None:
        from .workloads import make_config

        case = make_config(contract.config, seed=contract.seed)
    if grid_of is not None:
        refuse_noop_candidates(contract, case, grid_of)
    case_sha = hashlib.sha256(case.q.tobytes() + case.kv_pages.tobytes() + case.kv_lens.tobytes()
                              + case.page_indices.tobytes()).hexdigest()
    for pos, name in enumerate(contract.names):
        rel = f"gate/{pos:02d}-{name}"
        ensure_run(rel, name, save_output=True)
        if shared["input_sha256"] != case_sha:
            raise ValueError("RPA_SEARCH_INPUT_IDENTITY_MISMATCH: the checker's case is not the runs' input")
        verdict_path = root / rel / "correctness.json"
        if verdict_path.exists():
            verdict = json.loads(verdict_path.read_text())
        else:
            verdict = dict(checker(case, load_output(root / rel)))
            verdict_path.write_text(json.dumps(verdict, indent=1, sort_keys=True, default=float) + "\n")
            if not keep_outputs:
                (root / rel / "output.npy").unlink()
        gate[name] = verdict
    if not gate[contract.baseline].get("passed"):
        raise ValueError(f"RPA_SEARCH_BASELINE_FAILED_CORRECTNESS {gate[contract.baseline]}")
    active = [n for n in contract.names if gate[n].get("passed")]

    results = {n: [] for n in active}
    for r, order in enumerate(execution_orders(contract.names, contract.rounds)):
        for pos, name in enumerate(order):
            if name in results:
                results[name].append(ensure_run(f"round-{r:02d}/{pos:02d}-{name}", name))
    stats = statistics(contract, results)
    promotable = [n for n, s in stats.items() if s["promotable"]]
    winner = max(promotable, key=lambda n: stats[n]["improvement"]) if promotable else None
    confirmation = None
    if winner is not None and contract.confirmation_rounds:
        orders, base_runs, win_runs = [], [], []
        for r in range(contract.confirmation_rounds):
            order = (contract.baseline, winner) if r % 2 == 0 else (winner, contract.baseline)
            orders.append(order)
            for pos, name in enumerate(order):
                t = ensure_run(f"confirmation/round-{r:02d}/{pos:02d}-{name}", name)
                (base_runs if name == contract.baseline else win_runs).append(t)
        confirmation = confirmation_statistics(contract, winner, orders, base_runs, win_runs)
    confirmed = winner if confirmation is not None and confirmation["confirmed"] else None
    result = {"search_id": contract.search_id, "contract": contract.to_json(), "correctness": gate,
              "rejected_candidates": [n for n in contract.names if n not in active], "statistics": stats,
              "provisional_winner": winner, "confirmation": confirmation, "winner": confirmed,
              "winner_knobs": contract.knobs(confirmed) if confirmed else None,
              "incomplete_attempts": incomplete_attempts(root)}
    (root / "result.json").write_text(json.dumps(result, indent=1, sort_keys=True, default=float) + "\n")
    return result


def promote(result: dict, *, path=None) -> str | None:
    """Write a confirmed winner's knobs into the tuned table under its configuration's shape key;
    returns the key (None when nothing was confirmed)."""
    if not result.get("winner"):
        return None
    from .workloads import config_meta

    c = result["contract"]
    meta = config_meta(c["config"], seed=c["seed"])
    key = tuned.simplify_key("fp8" if c["config"] == "c4" else "bf16", meta.num_q_heads // meta.num_kv_heads,
                             meta.page_size, int(meta.q_lens.sum()))
    ci = result["confirmation"]["improvement_ci95"]
    tuned.write_entry(key, result["winner_knobs"], path=path, source=(
        f"knob search {result['search_id'][:16]} on {c['config']}: {result['winner']} over {c['baseline']}, "
        f"confirmed {result['confirmation']['improvement']:+.1%} [{ci[0]:+.1%}, {ci[1]:+.1%}]"))
    return key


def summary_markdown(result: dict, command: str) -> str:
    """A short summary of a search result (for profiles/): protocol, per-candidate statistics,
    confirmation and the correctness gate."""
    c = result["contract"]
    lines = [f"# Knob search on {c['config']} (search id {result['search_id'][:16]})", "",
             f"Command: `{command}`", "",
             f"Protocol: {len(c['candidates'])} candidates, {c['rounds']} rounds (forward + reversed Latin squares), "
             f"{c['confirmation_rounds']} confirmation rounds, {c['warmup']} warmup + {c['steps']} measured calls per "
             f"run, every run a rocprofv3-traced process (device time per call = the dispatches of its kernels), "
             f"paired per-round improvements, bootstrap 95% interval ({c['bootstrap_samples']} samples), "
             f"promotion above {c['minimum_practical_improvement']:.0%}.", "",
             "| candidate | knobs | gate max-abs | runs | median call (us) | paired improvement | 95% CI | promotable |",
             "|---|---|---|---|---|---|---|---|"]
    for name, knobs in c["candidates"]:
        gate = result["correctness"].get(name, {})
        st = result["statistics"].get(name)
        if st is None:
            lines.append(f"| {name} | {knobs} | {gate.get('max_abs', float('nan')):.2e} (rejected) | - | - | - | - | - |")
            continue
        lo, hi = st["improvement_ci95"]
        lines.append(f"| {name} | {knobs} | {gate.get('max_abs', float('nan')):.2e} | {st['runs']} | "
                     f"{st['median_ns'] / 1e3:.2f} | {st['improvement']:+.2%} | [{lo:+.2%}, {hi:+.2%}] | "
                     f"{'yes' if st['promotable'] else 'no'} |")
    conf = result.get("confirmation")
    lines += ["", f"Provisional winner: {result['provisional_winner']}; confirmed winner: {result['winner']}."]
    if conf:
        lo, hi = conf["improvement_ci95"]
        lines.append(f"Confirmation ({conf['runs']} paired rounds): {conf['improvement']:+.2%} [{lo:+.2%}, {hi:+.2%}].")
    return "\n".join(lines) + "\n"


def _parse_candidate(text: str):
    name, _, rest = text.partition(":")
    knobs = {}
    for item in filter(None, rest.split(",")):
        k, _, v = item.partition("=")
        if k not in KNOBS:
            raise ValueError(f"unknown knob {k!r} (knobs: {', '.join(KNOBS)})")
        knobs[k] = {"waves_per_cu": int, "prefill_cost": float, "prefill_tiles": int}[k](v)
    return name, knobs


def _load_checker(path: str):
    import importlib.util

    spec = importlib.util.spec_from_file_location("search_checker", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.oracle_checker


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m tpu_cake_amd.search")
    sub = ap.add_subparsers(dest="cmd")
    r = sub.add_parser("_run")
    r.add_argument("--config", required=True)
    r.add_argument("--knobs", required=True)
    r.add_argument("--steps", type=int, required=True)
    r.add_argument("--warmup", type=int, required=True)
    r.add_argument("--seed", type=int, default=None)
    r.add_argument("--out", required=True)
    r.add_argument("--save-output", action="store_true")
    ap.add_argument("--config", default="c3")
    ap.add_argument("--root")
    ap.add_argument("--checker", help="a Python file defining oracle_checker(case, output) (the correctness gate)")
    ap.add_argument("--candidate", action="append", help="name:knob=value,knob=value (the first is the baseline)")
    ap.add_argument("--rounds", type=int, default=0, help="default: two Latin squares")
    ap.add_argument("--confirmation-rounds", type=int, default=2)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=None)
    ap.add_argument("--bootstrap-samples", type=int, default=10_000)
    ap.add_argument("--promote", action="store_true", help="write a confirmed winner into the tuned table")
    ap.add_argument("--summary", help="also write a markdown summary of the result to this path")
    a = ap.parse_args(argv)
    if a.cmd == "_run":
        _child_run(a.config, json.loads(a.knobs), a.steps, a.warmup, pathlib.Path(a.out), a.seed, a.save_output)
        return 0
    if not (a.root and a.checker and a.candidate):
        ap.error("--root, --checker and --candidate are required")
    cands = tuple(_parse_candidate(c) for c in a.candidate)
    contract = SearchContract(config=a.config, baseline=cands[0][0], candidates=cands,
                              rounds=a.rounds or 2 * len(cands), confirmation_rounds=a.confirmation_rounds,
                              seed=a.seed, warmup=a.warmup, steps=a.steps, bootstrap_samples=a.bootstrap_samples)
    res = run_search(a.root, contract, runner=TraceRunner(), checker=_load_checker(a.checker))
    key = promote(res) if a.promote else None
    if a.summary:
        pathlib.Path(a.summary).write_text(summary_markdown(res, "python -m tpu_cake_amd.search " + " ".join(
            argv if argv is not None else sys.argv[1:])))
    print(json.dumps({"winner": res["winner"], "provisional_winner": res["provisional_winner"],
                      "rejected": res["rejected_candidates"], "promoted_key": key,
                      "medians_ns": {k: v["median_ns"] for k, v in res["statistics"].items()}}, sort_keys=True))
    return 0


if __name__ == "__main__":
    sys.exit(main())

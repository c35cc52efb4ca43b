"""Latin-square search over the RPA kernel's tuning knobs.

The reference searches Pallas block sizes (``src/tpu_cake/rpa_search.py:564-661``): each
candidate runs once per round, rounds follow forward and then reversed Latin squares of the
candidate list (every candidate takes every position equally often, so drift over a session
cancels, :201-210), per-candidate statistics decide a provisional winner over a baseline, and
confirmation rounds alternate the baseline and that winner.  The stream-K kernel here has no
block sizes -- its schedule balances work by itself -- so the searched parameters are its
run-time knobs, all read on every call: ``RPA_WAVES_PER_CU`` (the persistent grid),
``RPA_PF_COST`` (the prefill/decode work split) and ``RPA_NO_PREFILL_TILES``.  A candidate is
a name and the knob values it sets; a run is ``steps`` timed calls of one benchmark
configuration (HIP timing-only events around each call).

    python -m tpu_cake_amd.search --config c3 --root OUT \\
        --candidate base: --candidate pf25:RPA_PF_COST=0.25 --candidate pf50:RPA_PF_COST=0.5
"""

from __future__ import annotations

import argparse
import json
import math
import os
import pathlib
import random
import sys

KNOBS = ("RPA_WAVES_PER_CU", "RPA_PF_COST", "RPA_NO_PREFILL_TILES")


def execution_orders(names, rounds: int):
    """Round r runs the candidates rotated by r % n, in forward order in even squares and reversed
    order in odd squares (square = r // n)."""
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


def _median(xs):
    s = sorted(xs)
    n = len(s)
    return (s[n // 2] + s[(n - 1) // 2]) / 2


def _percentile(xs, q):
    s = sorted(xs)
    return s[min(len(s) - 1, round((len(s) - 1) * q))]


def statistics(runs: dict, baseline: str, *, resamples: int = 2000, seed: int = 0) -> dict:
    """runs: name -> list of per-run sample lists (ns).  Per candidate: run count, median of the
    run medians, p90 of the run medians, median absolute deviation and coefficient of variation
    of the run medians, improvement over the baseline (baseline median / candidate median - 1)
    with a bootstrap 95% interval over runs; promotable when the interval is above 0."""
    rng = random.Random(seed)
    meds = {k: [_median(r) for r in v] for k, v in runs.items()}
    base = meds[baseline]
    out = {}
    for name, m in meds.items():
        med = _median(m)
        mad = _median([abs(x - med) for x in m])
        mean = sum(m) / len(m)
        sd = math.sqrt(sum((x - mean) ** 2 for x in m) / max(1, len(m) - 1))
        boots = []
        for _ in range(resamples):
            b = [base[rng.randrange(len(base))] for _ in base]
            c = [m[rng.randrange(len(m))] for _ in m]
            boots.append(_median(b) / _median(c) - 1.0)
        boots.sort()
        lo, hi = boots[int(0.025 * resamples)], boots[int(0.975 * resamples) - 1]
        out[name] = {"runs": len(m), "samples": sum(len(r) for r in runs[name]), "median_ns": med,
                     "p90_run_median_ns": _percentile(m, 0.9), "mad_ns": mad, "cv": sd / mean if mean else 0.0,
                     "improvement": _median(base) / med - 1.0, "improvement_ci95": [lo, hi],
                     "promotable": name != baseline and lo > 0.0}
    return out


class _Runner:
    """One benchmark configuration resident on the GPU; run() times `steps` calls."""

    def __init__(self, config: str, seed=None):
        import torch

        from . import ops
        from .workloads import make_config

        self.torch, self.ops = torch, ops
        dev = torch.device("cuda", 0)
        self.case = make_config(config, seed=seed)
        self.d = ops.case_to_device(self.case, dev)
        pool = self.d["kv_pages"]
        self.copies = max(2, math.ceil(2e9 / (pool.numel() * pool.element_size())))
        self.pools = [pool] + [pool.clone() for _ in range(self.copies - 1)]
        self.kw = dict(sm_scale=self.case.sm_scale, out=self.torch.empty_like(self.d["q"]))
        if "kv_scales" in self.d:
            self.kw["kv_scales"] = self.d["kv_scales"]
        self.i = 0

    def run(self, env: dict, steps: int, warmup: int):
        from .timing import KernelEvent

        saved = {k: os.environ.get(k) for k in KNOBS}
        for k in KNOBS:
            os.environ.pop(k, None)
        os.environ.update(env)
        try:
            ev = [(KernelEvent(), KernelEvent()) for _ in range(steps)]
            d = self.d
            for t in range(warmup + steps):
                timed = t >= warmup
                if timed:
                    ev[t - warmup][0].record()
                self.ops.ragged_paged_attention(d["q"], self.pools[self.i % self.copies], d["kv_lens"],
                                                d["page_indices"], d["cu_q_lens"], d["num_seqs"], **self.kw)
                if timed:
                    ev[t - warmup][1].record()
                self.i += 1
            self.torch.cuda.synchronize()
            return [round(a.elapsed_time(b) * 1e6) for a, b in ev]
        finally:
            for k, v in saved.items():
                if v is None:
                    os.environ.pop(k, None)
                else:
                    os.environ[k] = v


def run_search(root, config: str, candidates: dict, *, baseline: str, rounds: int, steps: int = 20,
               warmup: int = 3, confirmation_rounds: int = 2, runner=None) -> dict:
    """candidates: name -> {knob: value}.  Writes ``root/result.json`` (and every run's samples
    under ``root/runs.json``) and returns the result."""
    for name, env in candidates.items():
        bad = set(env) - set(KNOBS)
        if bad:
            raise ValueError(f"candidate {name}: unknown knobs {sorted(bad)}")
    if baseline not in candidates:
        raise ValueError("the baseline must be one of the candidates")
    if confirmation_rounds % 2:
        raise ValueError("confirmation rounds must balance both run orders")
    root = pathlib.Path(root)
    root.mkdir(parents=True, exist_ok=True)
    runner = runner or _Runner(config)
    runs = {name: [] for name in candidates}
    log = []
    for r, order in enumerate(execution_orders(candidates, rounds)):
        for pos, name in enumerate(order):
            samples = runner.run(candidates[name], steps, warmup)
            runs[name].append(samples)
            log.append({"round": r, "position": pos, "candidate": name, "samples_ns": samples})
    interim = statistics(runs, baseline)
    promotable = [n for n, s in interim.items() if s["promotable"]]
    winner = min(promotable, key=lambda n: interim[n]["median_ns"]) if promotable else None
    if winner is not None:
        for r in range(confirmation_rounds):
            order = (baseline, winner) if r % 2 == 0 else (winner, baseline)
            for pos, name in enumerate(order):
                samples = runner.run(candidates[name], steps, warmup)
                runs[name].append(samples)
                log.append({"round": f"confirmation-{r}", "position": pos, "candidate": name, "samples_ns": samples})
    final = statistics(runs, baseline)
    confirmed = winner if winner is not None and final[winner]["promotable"] else None
    result = {"config": config, "baseline": baseline, "candidates": candidates, "rounds": rounds, "steps": steps,
              "warmup": warmup, "statistics": final, "provisional_winner": winner, "winner": confirmed}
    (root / "runs.json").write_text(json.dumps(log) + "\n")
    (root / "result.json").write_text(json.dumps(result, indent=1, sort_keys=True) + "\n")
    return result


def _parse_candidate(text: str):
    name, _, rest = text.partition(":")
    env = {}
    for item in filter(None, rest.split(",")):
        k, _, v = item.partition("=")
        env[k] = v
    return name, env


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m tpu_cake_amd.search")
    ap.add_argument("--config", default="c2")
    ap.add_argument("--root", required=True)
    ap.add_argument("--candidate", action="append", required=True,
                    help="name:KNOB=value,KNOB=value (the first is the baseline)")
    ap.add_argument("--rounds", type=int, default=0, help="default: two Latin squares")
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    a = ap.parse_args(argv)
    cands = dict(_parse_candidate(c) for c in a.candidate)
    rounds = a.rounds or 2 * len(cands)
    res = run_search(a.root, a.config, cands, baseline=next(iter(cands)), rounds=rounds, steps=a.steps,
                     warmup=a.warmup)
    print(json.dumps({"winner": res["winner"], "provisional_winner": res["provisional_winner"],
                      "medians_ns": {k: v["median_ns"] for k, v in res["statistics"].items()}}, sort_keys=True))
    return 0


if __name__ == "__main__":
    sys.exit(main())

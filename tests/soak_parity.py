"""Timed randomized parity soak (not collected by pytest: run it by name on a GPU box).

    PYTHONPATH=tpu-cake_amd:. python tests/soak_parity.py [--seed 11] [--seconds 150]

Three phases of --seconds each, every case against the CPU oracle at the bars of the committed
tests: the fused decode step over random shapes (page sizes 1-64 incl. ones that do not divide 32,
head dims 32-128, GQA 1-8, Hkv 1-16, R 0/16, bit-exact cache); prefill-heavy mixed batches over the
co-resident layout (test_gpu_random_sweep._prefill_heavy_case); and the general random batches
(test_gpu_random_sweep._random_case).  Prints each case before running it, then the case counts;
stops at the first case outside the bars and prints it with its max-abs against both oracles
(bf16 and fp32 probabilities), so a tolerance case can be told from a wrong result.
"""

import argparse
import importlib.util
import pathlib
import sys
import time

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent


def _load(name):
    spec = importlib.util.spec_from_file_location(name, HERE / f"{name}.py")
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def _check_operator(case, kw, desc):
    from oracle import rpa_oracle as orc
    from tpu_cake_amd import ops

    out = ops.run_case(case, **kw)
    torch.cuda.synchronize()
    out = out.float().cpu().numpy()
    args = (case.q, case.kv_pages, case.kv_lens, case.page_indices, case.cu_q_lens, case.num_seqs)
    common = dict(sm_scale=case.sm_scale, kv_scales=case.kv_scales, kv_dtype=case.kv_dtype, **kw)
    ref = orc.bf16_round(orc.ref_ragged_paged_attention(*args, probs_bf16=True, **common))
    got = out[: ref.shape[0]]
    small = np.abs(ref) < 4
    ok = (np.all(np.isfinite(got)) and np.allclose(got, ref, atol=0.02, rtol=0.02)
          and np.max(np.abs(got - ref)[small], initial=0.0) <= 2e-2)
    if not ok:
        ref32 = orc.ref_ragged_paged_attention(*args, probs_bf16=False, **common)
        print(f"OUTSIDE THE BARS: {desc}\n  max-abs vs bf16-probability oracle {np.max(np.abs(got - ref)):.3e}, "
              f"vs fp32-probability oracle {np.max(np.abs(got - ref32)):.3e}", flush=True)
    return ok


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--seed", type=int, default=11)
    ap.add_argument("--seconds", type=float, default=150.0)
    a = ap.parse_args()
    from oracle import rpa_fused_oracle as fo

    rs = _load("test_gpu_random_sweep")
    fz = _load("test_gpu_fused")
    rng = np.random.default_rng(a.seed)
    t0, n = time.time(), 0
    while time.time() - t0 < a.seconds:
        hkv = int(rng.choice([1, 2, 4, 8, 16]))
        g = int(rng.choice([1, 2, 4, 8]))
        page = int(rng.choice([1, 2, 3, 4, 8, 12, 16, 20, 24, 31, 32, 48, 64]))
        d = int(rng.choice([32, 40, 64, 96, 120, 128]))
        nseq = int(rng.integers(1, 30))
        lens = [int(x) for x in rng.integers(1, 2500, size=nseq)]
        lens[0] = int(rng.choice([1, 31, 32, 33, page, page + 1]))
        rel = int(rng.choice([0, 16]))
        extent = 8 * int(rng.integers(1, 80))
        pool = int(sum(-(-x // page) for x in lens) * 1.25) + 2
        print(f"[case] fused hq={hkv * g} hkv={hkv} d={d} page={page} nseq={nseq} R={rel} E={extent}", flush=True)
        inp = fo.fused_inputs_like(1000 + n, nseq=nseq, hq=hkv * g, hkv=hkv, d=d, page_size=page, pool_pages=pool,
                                   lengths=lens, rel_dim=rel, extent=extent)
        fz._run_and_check(inp)
        n += 1
    print(f"fused cases {n}", flush=True)
    for label, make in (("prefill-heavy", rs._prefill_heavy_case), ("random", rs._random_case)):
        t0, n = time.time(), 0
        while time.time() - t0 < a.seconds:
            case, kw, desc = make(rng)
            print(f"[case] {label} {desc}", flush=True)
            if not _check_operator(case, kw, desc):
                print(f"{label} cases {n} before it", flush=True)
                return 1
            n += 1
        print(f"{label} cases {n}", flush=True)
    print("SOAK OK", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

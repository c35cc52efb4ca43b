"""Run the three-phase evidence pipeline (tpu_cake_amd.evidence) with the oracle as the
correctness checker, and write a validated receipt.  Test infrastructure: the checker is the
oracle, which the package itself never imports.

    python tests/evidence_run.py --config c2 --root gpurun_out/evidence_c2 [--steps 10 --warmup 3]
"""

import argparse
import json
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[1]
sys.path[:0] = [str(ROOT), str(ROOT / "tpu-cake_amd")]

from oracle import rpa_oracle as orc  # noqa: E402
from tpu_cake_amd import evidence  # noqa: E402

TOL = 2e-2


def oracle_checker(case, out):
    """The reference's correctness gate (rpa_runner.py:105-122): max-abs against the oracle."""
    ref = orc.ref_ragged_paged_attention(case.q, case.kv_pages, case.kv_lens, case.page_indices, case.cu_q_lens,
                                         case.num_seqs, sm_scale=case.sm_scale, kv_scales=case.kv_scales,
                                         kv_dtype=case.kv_dtype)
    got = (out.float().cpu().numpy() if hasattr(out, "float") else np.asarray(out, np.float32))[: ref.shape[0]]
    err = orc.errors(got, orc.bf16_round(ref))
    return {"oracle": "oracle/rpa_oracle.py::ref_ragged_paged_attention", "tolerance": TOL,
            "max_abs": err["max_abs"], "max_rel": err["max_rel"], "rel_l2": err["rel_l2"], "finite": err["finite"],
            "passed": bool(err["finite"] and err["max_abs"] <= TOL)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="c2")
    ap.add_argument("--root", required=True)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    a = ap.parse_args()
    rec = evidence.run_all(a.root, a.config, a.steps, a.warmup, oracle_checker)
    print(json.dumps({"status": rec["status"], "reasons": rec["reasons"], "metrics": rec["metrics"]},
                     sort_keys=True), flush=True)
    return 0 if rec["status"] == "passed" else 1


if __name__ == "__main__":
    sys.exit(main())

"""Writes tests/golden/*.npz from the CPU oracle (run from the repo root).

c1_expected.npz: the C1 benchmark case (seeded generator) -- its metadata, a
sha256 of its q / kv_pages bytes, and the oracle's bf16 output.  The reference
ships no golden arrays for this path (its RPA tests hold only seeds, page-id
prefixes and known answers), so these vectors pin the build's own oracle and
generator against silent drift.
"""

import hashlib
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "tpu-cake_amd")]

from oracle import rpa_oracle as orc  # noqa: E402
from tpu_cake_amd.workloads import make_config  # noqa: E402


def main():
    case = make_config("c1", values="host")
    ref = orc.ref_ragged_paged_attention(case.q, case.kv_pages, case.kv_lens, case.page_indices, case.cu_q_lens,
                                         case.num_seqs, sm_scale=case.sm_scale)
    out = pathlib.Path(__file__).with_name("c1_expected.npz")
    np.savez_compressed(
        out,
        kv_lens=case.kv_lens, page_indices=case.page_indices, cu_q_lens=case.cu_q_lens,
        q_sha256=np.frombuffer(hashlib.sha256(case.q.tobytes()).digest(), np.uint8),
        kv_sha256=np.frombuffer(hashlib.sha256(case.kv_pages.tobytes()).digest(), np.uint8),
        out_bf16=orc.bf16_from_f32(ref),
    )
    print(out, ref.shape)


if __name__ == "__main__":
    main()

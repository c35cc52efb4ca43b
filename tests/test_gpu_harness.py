"""The evidence harness on the GPU: a knob search (tpu_cake_amd.search) and the timing phase with
the oracle as checker (tpu_cake_amd.evidence); the rocprofv3 phases run from tests/evidence_run.py."""

import json
import sys
import pathlib

import pytest
import torch

from tpu_cake_amd import evidence, search

sys.path.insert(0, str(pathlib.Path(__file__).resolve().parent))
import evidence_run  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def test_search_runs_every_candidate_in_latin_order(cuda, tmp_path):
    print("[case] knob search c1", flush=True)
    cands = {"base": {}, "w4": {"RPA_WAVES_PER_CU": "4"}}
    res = search.run_search(tmp_path, "c1", cands, baseline="base", rounds=4, steps=3, warmup=1)
    log = json.loads((tmp_path / "runs.json").read_text())
    assert [e["candidate"] for e in log[:4]] == ["base", "w4", "w4", "base"]
    for name in cands:
        st = res["statistics"][name]
        assert st["runs"] >= 2 and st["median_ns"] > 0
    assert res["winner"] in (None, "w4")


def test_timing_phase_with_the_oracle_checker(cuda, tmp_path):
    print("[case] evidence timing phase c1", flush=True)
    res = evidence.run_timing(tmp_path, "c1", 3, 1, checker=evidence_run.oracle_checker)
    assert res["passed"] and res["correctness"]["checked"] and res["correctness"]["max_abs"] <= 2e-2
    samples = json.loads((tmp_path / "timing" / "samples.json").read_text())
    assert len(samples["attention_ns"]) == 3 and min(samples["call_ns"]) >= min(samples["attention_ns"]) > 0
    assert res["identity"]["kernel_source_digest"] == evidence.kernel_source_digest()

"""The evidence harness on the GPU: a knob search (tpu_cake_amd.search) and the timing phase with
the oracle as checker (tpu_cake_amd.evidence); the rocprofv3 phases run from tests/evidence_run.py."""

import json
import pathlib
import sys

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


def test_search_with_trace_runs_and_the_oracle_gate(cuda, tmp_path):
    """A small real search on C1: every run a rocprofv3-traced child process, the objective from the
    trace, every candidate gated by the oracle; then a resume re-validates every run."""
    print("[case] knob search c1 (rocprofv3 runs)", flush=True)
    c = search.SearchContract(config="c1", baseline="base", candidates=(("base", {}), ("w4", {"waves_per_cu": 4})),
                              rounds=4, confirmation_rounds=0, steps=3, warmup=1, bootstrap_samples=1000)
    res = search.run_search(tmp_path, c, runner=search.TraceRunner(timeout_s=240), checker=evidence_run.oracle_checker)
    assert res["rejected_candidates"] == []
    assert all(v["passed"] and v["max_abs"] <= 2e-2 for v in res["correctness"].values())
    for name in ("base", "w4"):
        st = res["statistics"][name]
        assert st["runs"] == 4 and st["samples"] == 12 and st["median_ns"] > 0
    assert res["winner"] is None  # no confirmation rounds were asked for

    class NoRuns:
        def run(self, *a, **k):
            raise AssertionError("a completed run was run again")

    again = search.run_search(tmp_path, c, runner=NoRuns(), checker=evidence_run.oracle_checker)
    assert again["statistics"]["w4"]["median_ns"] == res["statistics"]["w4"]["median_ns"]


def test_timing_phase_with_the_oracle_checker(cuda, tmp_path):
    print("[case] evidence timing phase c1", flush=True)
    res = evidence.run_timing(tmp_path, "c1", 3, 1, checker=evidence_run.oracle_checker)
    assert res["passed"] and res["correctness"]["checked"] and res["correctness"]["max_abs"] <= 2e-2
    samples = json.loads((tmp_path / "timing" / "samples.json").read_text())
    assert len(samples["attention_ns"]) == 3 and min(samples["call_ns"]) >= min(samples["attention_ns"]) > 0
    assert res["identity"]["kernel_source_digest"] == evidence.kernel_source_digest()

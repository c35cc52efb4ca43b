"""The evidence harness on the CPU: the Latin-square execution orders and search statistics
(tpu_cake_amd.search, after rpa_search.py:201-210), rocprofv3 profile inspection and the receipt
over three phases (tpu_cake_amd.evidence, after rpa_bundle.py:664-800), on synthetic files."""

import json

import pytest

from tpu_cake_amd import evidence, search


def test_orders_are_forward_then_reversed_latin_squares():
    orders = search.execution_orders(["a", "b", "c"], 6)
    assert orders[:3] == (("a", "b", "c"), ("b", "c", "a"), ("c", "a", "b"))
    assert orders[3:] == (("c", "b", "a"), ("b", "a", "c"), ("a", "c", "b"))
    for pos in range(3):  # every candidate takes every position equally often
        assert sorted(o[pos] for o in orders) == ["a", "a", "b", "b", "c", "c"]
    with pytest.raises(ValueError, match="Latin squares"):
        search.execution_orders(["a", "b"], 3)


def test_statistics_promote_only_a_clear_improvement():
    base = [[100 + (i % 3)] * 5 for i in range(8)]
    fast = [[80 + (i % 3)] * 5 for i in range(8)]
    same = [[100 + ((i + 1) % 3)] * 5 for i in range(8)]
    st = search.statistics({"base": base, "fast": fast, "same": same}, "base", resamples=400)
    assert st["fast"]["promotable"] and st["fast"]["improvement"] > 0.2
    assert not st["same"]["promotable"] and not st["base"]["promotable"]
    assert st["base"]["runs"] == 8 and st["base"]["samples"] == 40


class _FakeRunner:
    def __init__(self, times):
        self.times = times
        self.calls = []

    def run(self, env, steps, warmup):
        self.calls.append(dict(env))
        return [self.times[env.get("RPA_PF_COST", "base")]] * steps


def test_search_confirms_a_winner(tmp_path):
    fake = _FakeRunner({"base": 100, "0.25": 90, "0.5": 120})
    cands = {"base": {}, "pf25": {"RPA_PF_COST": "0.25"}, "pf50": {"RPA_PF_COST": "0.5"}}
    res = search.run_search(tmp_path, "c3", cands, baseline="base", rounds=6, steps=3, warmup=0, runner=fake)
    assert res["winner"] == "pf25" and res["provisional_winner"] == "pf25"
    assert len(fake.calls) == 6 * 3 + 2 * 2  # the rounds, then two confirmation pairs
    assert json.loads((tmp_path / "result.json").read_text())["winner"] == "pf25"
    with pytest.raises(ValueError, match="unknown knobs"):
        search.run_search(tmp_path, "c3", {"x": {"BOGUS": "1"}}, baseline="x", rounds=2, runner=fake)


def _write_profile(d, attn_calls=10, counters=None):
    d.mkdir(parents=True, exist_ok=True)
    (d / "run_kernel_stats.csv").write_text(
        '"Name","Calls","TotalDurationNs","AverageNs","Percentage","MinNs","MaxNs","StdDev"\n'
        f'"void rpa::(anonymous namespace)::rpa_attn_kernel<0, true>(Params)",{attn_calls},{attn_calls * 1000},1000,90,900,1100,10\n'
        f'"rpa::(anonymous namespace)::rpa_combine_kernel(Params)",{attn_calls},{attn_calls * 100},100,9,90,110,1\n'
        '"__amd_rocclr_copyBuffer",3,300,100,1,90,110,1\n')
    if counters:
        rows = ['"Correlation_Id","Dispatch_Id","Kernel_Name","Counter_Name","Counter_Value"']
        for c, v in counters.items():
            for i in range(attn_calls):
                rows.append(f'{i},{i},"void rpa::(anonymous namespace)::rpa_attn_kernel<0, true>(Params)","{c}",'
                            f'{v + 2 * (i % 2)}')
                rows.append(f'{i},{100 + i},"rpa::(anonymous namespace)::rpa_combine_kernel(Params)","{c}",1')
        (d / "run_counter_collection.csv").write_text("\n".join(rows) + "\n")


def test_inspect_and_assess_profile(tmp_path):
    _write_profile(tmp_path / "t", counters={"FETCH_SIZE": 100.0})
    prof = evidence.inspect_profile(tmp_path / "t")
    assert prof["kernels"]["rpa_attn_kernel"]["calls"] == 10
    assert prof["kernels"]["rpa_attn_kernel"]["avg_ns"] == 1000
    assert "copyBuffer" not in json.dumps(prof["kernels"])
    assert prof["counters"]["rpa_attn_kernel"]["FETCH_SIZE"] == 101.0
    assert evidence.assess_profile(prof, dispatches=10)["accepted"]
    assert prof["counter_dispatches"]["rpa_attn_kernel"] == 10
    bad = evidence.assess_profile(prof, dispatches=11, counters=("FETCH_SIZE", "WRITE_SIZE"))
    assert not bad["accepted"] and len(bad["reasons"]) == 3


def _phase(root, mode, identity, passed=True, checked=True):
    d = root / mode
    if mode == "timing":
        d.mkdir(parents=True)
        (d / "samples.json").write_text(json.dumps({"attention_ns": [10, 12, 11], "call_ns": [20, 22, 21]}))
        body = {"correctness": {"checked": checked, "passed": passed, "max_abs": 0.004}, "passed": passed}
    else:
        _write_profile(d, counters={"FETCH_SIZE": 5.0, "WRITE_SIZE": 1.0} if mode == "counters" else None)
        prof = evidence.inspect_profile(d)
        ass = evidence.assess_profile(prof, dispatches=10, counters=evidence.COUNTERS if mode == "counters" else ())
        body = {"profile": prof, "assessment": ass, "passed": ass["accepted"]}
    arts = [{"path": str(p.relative_to(d)), "sha256": evidence.sha256_file(p), "role": "x"}
            for p in sorted(d.rglob("*")) if p.is_file()]
    res = {"mode": mode, "identity": identity, "config": "c1", "steps": 10, "input_sha256": "ab", **body,
           "artifacts": arts}
    (d / "result.json").write_text(json.dumps(res))


def test_receipt_passes_and_detects_tampering(tmp_path):
    ident = {"kernel_source_digest": "k", "library_sha256": "l"}
    for m in evidence.PHASES:
        _phase(tmp_path, m, ident)
    rec = evidence.build_receipt(tmp_path)
    assert rec["status"] == "passed", rec["reasons"]
    assert rec["metrics"]["timing.attention_median_ns"] == 11
    assert rec["metrics"]["trace.attention_avg_ns"] == 1000
    evidence.validate_receipt(tmp_path)
    (tmp_path / "trace" / "run_kernel_stats.csv").write_text("changed\n")
    with pytest.raises(ValueError, match="ARTIFACT_CHANGED"):
        evidence.validate_receipt(tmp_path)


@pytest.mark.parametrize("mutate,reason", [("identity", "disagree on identity"), ("unchecked", "not checked"),
                                           ("failed", "timing phase did not pass")])
def test_receipt_rejections(tmp_path, mutate, reason):
    ident = {"kernel_source_digest": "k", "library_sha256": "l"}
    _phase(tmp_path, "timing", ident, passed=mutate != "failed", checked=mutate != "unchecked")
    _phase(tmp_path, "trace", dict(ident, kernel_source_digest="other") if mutate == "identity" else ident)
    _phase(tmp_path, "counters", ident)
    rec = evidence.build_receipt(tmp_path)
    assert rec["status"] == "rejected" and any(reason in r for r in rec["reasons"]), rec["reasons"]

"""The evidence harness on the CPU: the Latin-square execution orders and search statistics
(tpu_cake_amd.search, after rpa_search.py:201-210), rocprofv3 profile inspection and the receipt
over three phases (tpu_cake_amd.evidence, after rpa_bundle.py:664-800), on synthetic files."""

import hashlib
import json

import numpy as np
import pytest

from tpu_cake_amd import evidence, search, tuned


def test_orders_are_forward_then_reversed_latin_squares():
    orders = search.execution_orders(["a", "b", "c"], 6)
    assert orders[:3] == (("a", "b", "c"), ("b", "c", "a"), ("c", "a", "b"))
    assert orders[3:] == (("c", "b", "a"), ("b", "a", "c"), ("a", "c", "b"))
    for pos in range(3):  # every candidate takes every position equally often
        assert sorted(o[pos] for o in orders) == ["a", "a", "b", "b", "c", "c"]
    with pytest.raises(ValueError, match="Latin squares"):
        search.execution_orders(["a", "b"], 3)


def _contract(**kw):
    base = dict(config="c3", baseline="incumbent", rounds=6, confirmation_rounds=6, bootstrap_samples=1000,
                candidates=(("incumbent", {}), ("pf25", {"prefill_cost": 0.25}), ("pf50", {"prefill_cost": 0.5})))
    base.update(kw)
    return search.SearchContract(**base)


def _timing(median):
    return search.DeviceTiming.of([float(median)] * 50)


def test_statistics_promote_from_paired_run_level_measurements():
    # the reference's own case (tests/test_rpa_search.py:100-115): 20% faster in every round is
    # promotable with an interval above the 1% practical threshold, +-2% noise is not
    c = _contract()
    res = {"incumbent": [_timing(v) for v in (100, 102, 98, 101, 99, 100)],
           "pf25": [_timing(v) for v in (80, 82, 78, 81, 79, 80)],
           "pf50": [_timing(v) for v in (101, 100, 100, 102, 99, 101)]}
    st = search.statistics(c, res)
    assert st["pf25"]["promotable"] and st["pf25"]["runs"] == 6 and st["pf25"]["samples"] == 300
    assert st["pf25"]["improvement_ci95"][0] > 0.01
    assert not st["pf50"]["promotable"] and not st["incumbent"]["promotable"]


def test_statistics_are_paired_per_round():
    # a session-wide drift that hits both candidates alike: unpaired medians overlap, the paired
    # per-round improvement (always +3%) is promotable
    c = _contract(candidates=(("incumbent", {}), ("pf25", {"prefill_cost": 0.25})), rounds=8)
    drift = [100, 130, 90, 120, 95, 140, 105, 110]
    res = {"incumbent": [_timing(d) for d in drift], "pf25": [_timing(d * 0.97) for d in drift]}
    st = search.statistics(c, res)
    assert st["pf25"]["promotable"] and abs(st["pf25"]["improvement"] - 0.03) < 1e-9
    # below the practical threshold: +0.5% every round is real but not worth promoting
    res = {"incumbent": [_timing(d) for d in drift], "pf25": [_timing(d * 0.995) for d in drift]}
    assert not search.statistics(c, res)["pf25"]["promotable"]


def test_confirmation_requires_fresh_paired_improvement():
    c = _contract()
    orders = [("incumbent", "pf25") if i % 2 == 0 else ("pf25", "incumbent") for i in range(6)]
    conf = search.confirmation_statistics(c, "pf25", orders, [_timing(v) for v in (100, 102, 98, 101, 99, 100)],
                                          [_timing(v) for v in (80, 82, 78, 81, 79, 80)])
    assert conf["confirmed"] and conf["runs"] == 6 and conf["orders"][1] == ["pf25", "incumbent"]
    conf = search.confirmation_statistics(c, "pf25", orders, [_timing(100)] * 6, [_timing(99.5)] * 6)
    assert not conf["confirmed"]


@pytest.mark.parametrize("kw,msg", [(dict(rounds=4), "Latin squares"), (dict(confirmation_rounds=3), "both run orders"),
                                    (dict(baseline="nope"), "baseline"),
                                    (dict(candidates=(("a", {}), ("b", {"prefill_cost": 0.0}))), "unique"),
                                    (dict(candidates=(("a", {}), ("b", {"bogus": 1}))), "unknown knobs"),
                                    (dict(bootstrap_samples=10), "bootstrap")])
def test_contract_rejections(kw, msg):
    if "candidates" in kw:
        kw.setdefault("baseline", "a")
        kw.setdefault("rounds", 4)
    with pytest.raises(ValueError, match=msg):
        _contract(**kw)


def _trace_csv(path, durations_by_call):
    """A kernel trace of calls given as (attention, prefill, combine) durations (0: not dispatched)."""
    path.parent.mkdir(parents=True, exist_ok=True)
    rows = ['"Kind","Dispatch_Id","Kernel_Name","Start_Timestamp","End_Timestamp"']
    names = ("void rpa::(anonymous namespace)::rpa_attn_kernel<0, true>(Params)",
             "rpa::(anonymous namespace)::rpa_prefill_kernel(Params)",
             "rpa::(anonymous namespace)::rpa_combine_kernel(Params)")
    t, did = 1000, 0
    for i, durs in enumerate(durations_by_call):
        for name, d in zip(names, durs):
            if d:
                rows.append(f'"KERNEL_DISPATCH",{did},"{name}",{t},{t + d}')
                did += 1
                t += d + 7
        rows.append(f'"KERNEL_DISPATCH",{900 + i},"__amd_rocclr_copyBuffer",{t},{t + 3}')
        t += 50
    path.write_text("\n".join(rows) + "\n")


def test_device_timing_from_the_kernel_trace(tmp_path):
    _trace_csv(tmp_path / "trace" / "x" / "run_kernel_trace.csv", [(500, 0, 50)] * 2 + [(100 + i, 0, 10) for i in range(4)])
    t = search.device_timing(tmp_path, 4)  # the last 4 calls, attention + combine each
    assert t.durations_ns == (110.0, 111.0, 112.0, 113.0) and t.median_ns == 111.5
    with pytest.raises(ValueError, match="DISPATCH_PROTOCOL"):
        search.device_timing(tmp_path, 7)
    # calls with the prefill kernel: attention + prefill + combine each
    _trace_csv(tmp_path / "pk" / "run_kernel_trace.csv", [(100 + i, 40, 10) for i in range(3)])
    assert search.device_timing(tmp_path / "pk", 3).durations_ns == (150.0, 151.0, 152.0)
    # calls that dispatch different kernel sequences are not one protocol
    _trace_csv(tmp_path / "mix" / "run_kernel_trace.csv", [(100, 0, 10), (100, 40, 10)])
    with pytest.raises(ValueError, match="DISPATCH_PROTOCOL"):
        search.device_timing(tmp_path / "mix", 2)


def test_incomplete_run_is_archived_with_a_manifest(tmp_path):
    run = tmp_path / "round-00" / "00-incumbent"
    run.mkdir(parents=True)
    (run / "failure.log").write_text("launch failed\n")
    arch = search.archive_incomplete_run(tmp_path, run, "launch failed")
    assert not run.exists() and arch == tmp_path / "incomplete/round-00/00-incumbent-attempt-00"
    assert "launch failed" in (arch / "failure.json").read_text()
    att = search.incomplete_attempts(tmp_path)
    assert len(att) == 1 and att[0]["path"] == "incomplete/round-00/00-incumbent-attempt-00"
    before = att[0]["manifest_sha256"]
    (arch / "failure.log").write_text("changed\n")
    assert search.incomplete_attempts(tmp_path)[0]["manifest_sha256"] != before
    run.mkdir(parents=True)
    assert search.archive_incomplete_run(tmp_path, run, "again").name == "00-incumbent-attempt-01"


class _Case:
    def __init__(self):
        self.q = np.arange(8, dtype=np.uint16)
        self.kv_pages = np.arange(16, dtype=np.uint16)
        self.kv_lens = np.array([3], np.int32)
        self.page_indices = np.array([[0]], np.int32)

    def sha(self):
        return hashlib.sha256(self.q.tobytes() + self.kv_pages.tobytes() + self.kv_lens.tobytes()
                              + self.page_indices.tobytes()).hexdigest()


class _FakeRunner:
    """Writes what a TraceRunner run leaves: steps.json, output.npy and a kernel trace; the device
    time per call depends on the candidate's prefill_cost, its output bits on whether it is 'bad'."""

    def __init__(self, case, times):
        self.case, self.times, self.calls = case, times, []

    def run(self, run_root, contract, knobs, save_output=False):
        self.calls.append(str(run_root))
        run_root.mkdir(parents=True, exist_ok=True)
        cost = knobs["prefill_cost"]
        out = np.full(4, 7 if cost != 0.7 else 9, np.uint16)
        (run_root / "steps.json").write_text(json.dumps({
            "identity": {"kernel_source_digest": "k", "library_sha256": "l"}, "input_sha256": self.case.sha(),
            "config": contract.config, "knobs": knobs, "output_sha256": hashlib.sha256(out.tobytes()).hexdigest()}))
        if save_output:
            np.save(run_root / "output.npy", out)
        n = len(self.calls)
        _trace_csv(run_root / "trace" / "h" / "run_kernel_trace.csv",
                   [(self.times[cost] + (n % 3), 0, 10)] * (contract.warmup + contract.steps))


def _checker(case, out):
    return {"passed": bool(np.all(out == out[0]) and out[0] != 0 and
                           np.all(out.view(np.uint32) >> 16 == 7)), "max_abs": 0.0}


def test_search_gates_times_confirms_and_resumes(tmp_path):
    case = _Case()
    c = _contract(candidates=(("incumbent", {}), ("pf25", {"prefill_cost": 0.25}), ("pf50", {"prefill_cost": 0.5}),
                              ("bad", {"prefill_cost": 0.7})), rounds=8, confirmation_rounds=2, steps=5, warmup=2)
    fake = _FakeRunner(case, {0.0: 1000, 0.25: 900, 0.5: 1200, 0.7: 500})
    res = search.run_search(tmp_path, c, runner=fake, checker=_checker, case=case)
    # 'bad' (fastest, wrong output) fails the gate and is never timed
    assert res["rejected_candidates"] == ["bad"] and not res["correctness"]["bad"]["passed"]
    assert not any("round-" in p and p.endswith("-bad") for p in fake.calls)
    assert res["provisional_winner"] == "pf25" and res["winner"] == "pf25"
    assert res["winner_knobs"]["prefill_cost"] == 0.25 and res["confirmation"]["confirmed"]
    assert len(fake.calls) == 4 + 8 * 3 + 2 * 2
    assert json.loads((tmp_path / "result.json").read_text())["winner"] == "pf25"
    # resume: every run re-validated from its files, nothing re-run
    fake.calls.clear()
    assert search.run_search(tmp_path, c, runner=fake, checker=_checker, case=case)["winner"] == "pf25"
    assert fake.calls == []
    # an unfinished run is archived and run again
    (tmp_path / "round-00" / "02-pf50" / "result.json").unlink()
    search.run_search(tmp_path, c, runner=fake, checker=_checker, case=case)
    assert fake.calls == [str(tmp_path / "round-00" / "02-pf50")]
    assert search.incomplete_attempts(tmp_path)[0]["path"] == "incomplete/round-00/02-pf50-attempt-00"
    # a tampered timing no longer replays; a changed contract is refused
    tpath = tmp_path / "round-00" / "00-incumbent" / "device_timing.json"
    tpath.write_text(tpath.read_text().replace('"median_ns": 1', '"median_ns": 2'))
    with pytest.raises(ValueError, match="REPLAY_MISMATCH"):
        search.run_search(tmp_path, c, runner=fake, checker=_checker, case=case)
    with pytest.raises(ValueError, match="CONTRACT_CHANGED"):
        search.run_search(tmp_path, _contract(rounds=12), runner=fake, checker=_checker, case=case)


def test_search_refuses_a_candidate_whose_output_changes(tmp_path):
    case = _Case()
    c = _contract(candidates=(("incumbent", {}), ("pf25", {"prefill_cost": 0.25})), rounds=4, confirmation_rounds=0,
                  steps=3, warmup=0)

    class Flaky(_FakeRunner):
        def run(self, run_root, contract, knobs, save_output=False):
            super().run(run_root, contract, knobs, save_output)
            if "round-01" in str(run_root) and knobs["prefill_cost"] == 0.25:
                st = json.loads((run_root / "steps.json").read_text())
                st["output_sha256"] = hashlib.sha256(np.full(4, 8, np.uint16).tobytes()).hexdigest()
                (run_root / "steps.json").write_text(json.dumps(st))

    with pytest.raises(ValueError, match="CANDIDATE_OUTPUT_MISMATCH"):
        search.run_search(tmp_path, c, runner=Flaky(case, {0.0: 100, 0.25: 90}), checker=_checker, case=case)
    assert search.incomplete_attempts(tmp_path)  # the offending run was archived


def test_promote_writes_the_tuned_table(tmp_path):
    res = {"winner": "pf25", "winner_knobs": {"waves_per_cu": 0, "prefill_tiles": True, "prefill_cost": 0.25},
           "search_id": "ab" * 32, "contract": {"config": "c3", "seed": None, "baseline": "incumbent"},
           "confirmation": {"improvement": 0.05, "improvement_ci95": [0.02, 0.08]}}
    path = tmp_path / "tuned.json"
    key = search.promote(res, path=path)
    assert key == "bf16/g4/p64/t4096"
    assert tuned.get_tuned_knobs("bf16", 4, 64, 2072, path=path)["prefill_cost"] == 0.25
    assert tuned.get_tuned_knobs("bf16", 4, 64, 64, path=path) == tuned.DEFAULTS
    assert search.promote(dict(res, winner=None), path=path) is None


def test_tuned_table_keys_and_checked_in_entries():
    assert tuned.simplify_key("bf16", 4, 64, 2072) == "bf16/g4/p64/t4096"
    assert tuned.simplify_key("fp8", 3, 24, 1) == "fp8/g4/p32/t1"
    with pytest.raises(ValueError):
        tuned.validate_entry({"waves_per_cu": 9})
    for key, entry in tuned.table().items():  # the checked-in table is valid
        assert entry == tuned.validate_entry(entry) and key.count("/") == 3


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


def test_receipt_mfma_fraction_and_markdown(tmp_path):
    ident = {"kernel_source_digest": "k", "library_sha256": "l"}
    for m in ("timing", "trace"):
        _phase(tmp_path, m, ident)
    # the counters phase with the MFMA counters: 2.56e6 busy cycles over 1024 SIMDs against 8e4 GUI-active
    # cycles summed over 8 XCD instances (1e4 per XCD) is a busy fraction of 2.56e6 / (1e4 * 1024) = 0.25
    d = tmp_path / "counters"
    _write_profile(d, counters={"FETCH_SIZE": 5.0, "WRITE_SIZE": 1.0, "SQ_VALU_MFMA_BUSY_CYCLES": 2.56e6 - 1,
                                "GRBM_GUI_ACTIVE": 8e4 - 1, "SQ_INSTS_VALU_MFMA_MOPS_BF16": 10.0})
    prof = evidence.inspect_profile(d)
    ass = evidence.assess_profile(prof, dispatches=10, counters=evidence.COUNTERS + evidence.MFMA_COUNTERS)
    arts = [{"path": str(p.relative_to(d)), "sha256": evidence.sha256_file(p), "role": "x"}
            for p in sorted(d.rglob("*")) if p.is_file()]
    (d / "result.json").write_text(json.dumps({"mode": "counters", "identity": ident, "config": "c1", "steps": 10,
                                               "input_sha256": "ab", "profile": prof, "assessment": ass,
                                               "passed": ass["accepted"], "artifacts": arts}))
    rec = evidence.build_receipt(tmp_path)
    assert rec["status"] == "passed", rec["reasons"]
    assert rec["metrics"]["counters.attention_mfma_busy_fraction"] == 0.25
    md = evidence.receipt_markdown(tmp_path, "python tests/evidence_run.py --config c1 --root R")
    assert md.startswith("# Evidence receipt: C1 (timing, trace, counters)")
    assert "Status: **passed**" in md and "digest k." in md
    assert "| counters.attention_mfma_busy_fraction | 0.25 |" in md
    assert "Assessments: counters: accepted; trace: accepted" in md


@pytest.mark.parametrize("mutate,reason", [("identity", "disagree on identity"), ("unchecked", "not checked"),
                                           ("failed", "timing phase did not pass")])
def test_receipt_rejections(tmp_path, mutate, reason):
    ident = {"kernel_source_digest": "k", "library_sha256": "l"}
    _phase(tmp_path, "timing", ident, passed=mutate != "failed", checked=mutate != "unchecked")
    _phase(tmp_path, "trace", dict(ident, kernel_source_digest="other") if mutate == "identity" else ident)
    _phase(tmp_path, "counters", ident)
    rec = evidence.build_receipt(tmp_path)
    assert rec["status"] == "rejected" and any(reason in r for r in rec["reasons"]), rec["reasons"]


def _fake_raw(root):
    """Raw outputs of a profile run for C2 and the copy calibration, shaped like rocprofv3's CSVs."""
    attn = "void rpa::(anonymous namespace)::rpa_attn_kernel<0, true>(rpa::Params)"
    comb = "rpa::(anonymous namespace)::rpa_combine_kernel(rpa::Params)"
    copyk = "__amd_rocclr_copyBuffer"
    d = root / "prof_c2"
    d.mkdir(parents=True)
    (d / "c2_kernel_stats.csv").write_text(
        '"Name","Calls","TotalDurationNs","AverageNs","Percentage","MinNs","MaxNs","StdDev"\n'
        f'"{attn}",23,2367000,102913.0,90,99000,124000,10\n"{comb}",23,123000,5347.8,9,4800,6600,1\n')
    (root / "prof_c2.out").write_text('[bench] x\n{"attn_kernel_ms": {"avg": 0.1076}, "ms_per_step": 0.1183}\n')

    def cc(name, rows):
        (root / name).mkdir(parents=True)
        lines = ['"Correlation_Id","Dispatch_Id","Kernel_Name","Counter_Name","Counter_Value"']
        ncounters = len({c for _, c, _ in rows})
        for i, (k, c, v) in enumerate(rows):  # one row per (dispatch, counter)
            lines.append(f'{i},{i // ncounters},"{k}","{c}",{v}')
        (root / name / "run_counter_collection.csv").write_text("\n".join(lines) + "\n")

    cc("fetch_c2", [(attn, "FETCH_SIZE", 307979.0)] * 5)
    cc("write_c2", [(attn, "WRITE_SIZE", 5090.0)] * 5)
    cc("tcc_c2", [(attn, "TCC_EA0_RDREQ_128B_sum", 4924078.0), (attn, "TCC_EA0_RDREQ_64B_sum", 3598.0),
                  (attn, "TCC_EA0_RDREQ_32B_sum", 0.0), (attn, "TCC_EA0_WRREQ_64B_sum", 81000.0)])
    cc("mfma_c2", [(attn, "SQ_VALU_MFMA_BUSY_CYCLES", 2.0e7), (attn, "GRBM_GUI_ACTIVE", 2.1e5),
                   (attn, "SQ_INSTS_VALU_MFMA_MOPS_BF16", 1.2e5)])
    cc("fetch_copy", [(copyk, "FETCH_SIZE", 524288.0)] * 6)
    cc("write_copy", [(copyk, "WRITE_SIZE", 1048576.0)] * 6)


def test_profile_summaries_regenerate_identically(tmp_path):
    from tpu_cake_amd import profiling

    raw = tmp_path / "raw"
    _fake_raw(raw)
    a, b = tmp_path / "a", tmp_path / "b"
    t1 = profiling.summarize(raw, a, raw_label="gpurun_out/prof")
    profiling.summarize(raw, b, raw_label="gpurun_out/prof")
    for f in sorted(p.name for p in a.iterdir()):
        assert (a / f).read_bytes() == (b / f).read_bytes(), f
    assert sorted(p.name for p in a.iterdir()) == ["pmc_traffic.json", "rpa_attn_c2.md"]
    c2 = t1["configs"]["c2"]
    assert t1["fetch_factor"] == 2.0 and t1["write_factor"] == 1.0
    assert c2["traffic_bytes"] == round(307979.0 * 1024 * 2 + 5090.0 * 1024)
    assert c2["mfma"]["mfma_busy_fraction"] == round(2.0e7 / (2.1e5 / 8 * 1024), 4)
    md = (a / "rpa_attn_c2.md").read_text()
    assert "rocprofv3 --kernel-trace --stats -d gpurun_out/prof/prof_c2" in md and "| rpa_attn_kernel | 23 | 102.91" in md


def test_search_summary_markdown(tmp_path):
    case = _Case()
    c = _contract(candidates=(("incumbent", {}), ("pf25", {"prefill_cost": 0.25})), rounds=4, confirmation_rounds=2,
                  steps=3, warmup=0)
    res = search.run_search(tmp_path, c, runner=_FakeRunner(case, {0.0: 100, 0.25: 90}), checker=_checker, case=case)
    md = search.summary_markdown(res, "python -m tpu_cake_amd.search ...")
    assert "| pf25 |" in md and "confirmed winner: pf25" in md and "Confirmation (2 paired rounds)" in md

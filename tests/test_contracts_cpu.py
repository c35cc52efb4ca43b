"""Workload contracts (``render-workload`` / ``experiment``) on the CPU.

The experiment id and schedule hash are recomputed independently from the artifacts, the launch
plan's stream-K unit counts are recounted row by row, and the contracts' tensors are checked
against the generated benchmark cases."""

from __future__ import annotations

import hashlib
import json
import math
import pathlib
import re

import numpy as np
import pytest

from tpu_cake_amd import contracts
from tpu_cake_amd.workloads import config_meta, make_config

ROOT = pathlib.Path(__file__).resolve().parent.parent
KERNEL_SRC = (ROOT / "tpu-cake_amd" / "csrc" / "rpa_kernels.hip").read_text()


@pytest.mark.parametrize("name", sorted(contracts.WORKLOADS))
def test_artifacts_are_deterministic_and_self_consistent(name):
    text = contracts.render_workload(name)
    assert text == contracts.render_workload(name)
    exp = contracts.experiment(name)
    assert exp.schedule_sha256 == hashlib.sha256(text.encode()).hexdigest()
    art = json.loads(contracts.experiment_artifact_json(exp))
    # the id is sha256 of the artifact without it: sorted keys, compact separators
    body = dict(art)
    ident = body.pop("experiment_id")
    assert ident == hashlib.sha256(json.dumps(body, sort_keys=True, separators=(",", ":")).encode()).hexdigest()
    # the artifact parses back into the same experiment
    again = contracts.KernelExperiment.model_validate(body)
    assert again.experiment_id == ident
    assert exp.target.accelerator == "MI355X" and exp.target.chip_count == 1
    # every kernel the profile requires is a kernel of the library
    for k in exp.profile.required_timed_hlo_markers:
        assert re.search(rf"__global__[^\n]*\b{k}\(", KERNEL_SRC), k
    for src in exp.workload.execution.source_manifest:
        assert src.sha256 == hashlib.sha256((ROOT / src.path).read_bytes()).hexdigest()


# The reference's checked-in artifacts for its own row (data: sha256 of the files and the id they
# carry): examples/inkling-rpa.mlir and contracts/inkling-rpa-experiment.json.
REF_SCHEDULE_SHA256 = "b97d16b523329ed57890184ad9d6b0ed893d3c666874e919ccf857aa6591f4cc"
REF_EXPERIMENT_ID = "b288837a2a06fc716e66c3508f761d0d4d01e110df248dadb9fa542b31296932"
REF_EXPERIMENT_FILE_SHA256 = "9e098004545330efb41513a9b436a8c5f651e46768467f086638f41e3c351717"
# The reference's id formula (src/tpu_cake/contracts.py:214-224) hashes the profile's
# minimum_counter_device_planes (default 0, :105), which the checked-in artifact predates: the
# id its current code gives the same experiment.
REF_FORMULA_EXPERIMENT_ID = "6f641a51af96c717cbe33ade0300c1736395ceed59824536603e72e5f074180f"


def test_reference_inkling_rpa_row_reproduces_the_reference_artifacts(tmp_path, capsys):
    """render-workload / experiment inkling-rpa print the reference's TPU7x schedule text and
    experiment JSON byte for byte (its CLI's two outputs, src/tpu_cake/cli.py:655-676)."""
    text = contracts.render_workload("inkling-rpa")
    assert hashlib.sha256(text.encode()).hexdigest() == REF_SCHEDULE_SHA256
    exp = contracts.experiment("inkling-rpa")
    assert exp.schedule_sha256 == REF_SCHEDULE_SHA256
    assert exp.experiment_id == REF_FORMULA_EXPERIMENT_ID
    assert contracts.artifact_id(exp, checked_in_form=True) == REF_EXPERIMENT_ID
    out = tmp_path / "exp.json"
    assert contracts.main(["experiment", "inkling-rpa", "--checked-in-form", "--output", str(out)]) == 0
    assert f"EXPERIMENT_WRITTEN workload=inkling-rpa id={REF_EXPERIMENT_ID}" in capsys.readouterr().out
    assert hashlib.sha256(out.read_bytes()).hexdigest() == REF_EXPERIMENT_FILE_SHA256
    # the default form carries the field and the reference formula's id
    assert contracts.main(["experiment", "inkling-rpa", "--output", str(out)]) == 0
    assert f"EXPERIMENT_WRITTEN workload=inkling-rpa id={REF_FORMULA_EXPERIMENT_ID}" in capsys.readouterr().out
    assert json.loads(out.read_text())["profile"]["minimum_counter_device_planes"] == 0
    assert exp.target.accelerator == "TPU7x" and exp.workload.execution is None
    # a change to the schedule changes both hashes
    assert hashlib.sha256(text.replace("kv_block_size = #builtin.int<8>", "kv_block_size = #builtin.int<16>")
                          .encode()).hexdigest() != REF_SCHEDULE_SHA256


def test_ids_differ_between_workloads_and_follow_content():
    ids = {n: contracts.experiment(n).experiment_id for n in contracts.ALL_WORKLOADS}
    assert len(set(ids.values())) == len(ids)
    exp = contracts.experiment("mi355x-rpa-c2")
    changed = exp.model_copy(update={"benchmark": exp.benchmark.model_copy(update={"measured_iterations": 51})})
    assert changed.experiment_id != exp.experiment_id


@pytest.mark.parametrize("cfg", ["c1", "c2", "c3", "c4", "c5"])
def test_operator_contract_tensors(cfg):
    exp = contracts.experiment(f"mi355x-rpa-{cfg}")
    m = config_meta(cfg)
    t = {x.name: x for x in exp.workload.inputs}
    assert t["q"].shape == (int(np.sum(m.q_lens)), m.num_q_heads, 128)
    assert t["kv_pages"].shape == (m.pool_pages, m.page_size, 2 * m.num_kv_heads, 128)
    assert t["page_indices"].shape == (len(m.kv_lens), m.pages_per_seq)
    assert t["cu_q_lens"].shape == (len(m.kv_lens) + 1,)
    assert (t["kv_pages"].dtype == "f8e4m3") == (cfg == "c4") and (("kv_scales" in t) == (cfg == "c4"))
    assert exp.workload.stage.value == ("mixed" if cfg == "c3" else "steady_decode")
    assert exp.workload.outputs[0].shape == t["q"].shape


def test_config_meta_matches_generated_case():
    case = make_config("c1", values="host")
    m = config_meta("c1")
    assert np.array_equal(case.kv_lens, m.kv_lens)
    assert case.kv_pages.shape[0] == m.pool_pages and case.page_indices.shape[1] == m.pages_per_seq
    assert m.kv_read_bytes() == case.kv_read_bytes()


def _units_by_rows(kv_len, q_len, group):
    """Stream-K units recounted from the rows: a 16-row block visits the keys its last row sees."""
    rows = q_len * group
    units = 0
    for r0 in range(0, rows, 16):
        last_tok = (min(r0 + 15, rows - 1)) // group
        visible = kv_len - q_len + last_tok + 1
        units += math.ceil(visible / 32)
    return units


@pytest.mark.parametrize("cfg", ["c1", "c2", "c5"])
def test_plan_unit_counts(cfg):
    m = config_meta(cfg)
    group = m.num_q_heads // m.num_kv_heads
    hg = max(g for g in range(1, min(m.num_kv_heads, 8) + 1) if m.num_kv_heads % g == 0)
    W = sum(_units_by_rows(int(L), int(q), group) for L, q in zip(m.kv_lens, m.q_lens)) * (m.num_kv_heads // hg)
    text = contracts.render_workload(f"mi355x-rpa-{cfg}")
    assert f"stream-K = {W} units" in text
    grid = 256 * (8 // hg)
    lo, hi = W // grid, -(-W // grid)
    assert f"({lo}..{hi} units each)" in text


def test_plan_lds_matches_kernel_constants():
    # the per-wave LDS the host requests, restated from the kernel's own constants
    const = {k: int(v) for k, v in re.findall(r"constexpr int (kD|KV_CHUNK) = (\d+);",
                                               KERNEL_SRC + (ROOT / "tpu-cake_amd" / "csrc" / "rpa_schedule.h").read_text())}
    assert re.search(r"constexpr int kKtRow = kD \* 2 \+ 16;", KERNEL_SRC)
    assert re.search(r"constexpr int kVRow = kD \* 2 \+ 32;", KERNEL_SRC)
    assert re.search(r"constexpr int kVtBytes_ = KV_CHUNK \* kVRow;", KERNEL_SRC)
    assert re.search(r"constexpr int kKtBytes = KV_CHUNK \* kKtRow;", KERNEL_SRC)
    per_wave = const["KV_CHUNK"] * (const["kD"] * 2 + 32) + const["KV_CHUNK"] * (const["kD"] * 2 + 16)
    assert contracts.WAVE_LDS_BYTES == per_wave
    assert f"LDS {8 * per_wave} B" in contracts.render_workload("mi355x-rpa-c2")
    assert "whole 128-byte K/V lines" in contracts.render_workload("mi355x-rpa-c2")
    assert "16-byte operand loads" in contracts.render_workload("mi355x-rpa-c4")


def test_combine_grid_matches_kernel_constants():
    sched = (ROOT / "tpu-cake_amd" / "csrc" / "rpa_schedule.h").read_text()
    const = dict(re.findall(r"constexpr int (kHeavyContrib|kHeavySlices) = (\d+);", sched))
    assert int(const["kHeavyContrib"]) == contracts.HEAVY_CONTRIB
    assert int(const["kHeavySlices"]) == contracts.HEAVY_SLICES
    # 256 workgroups of 8 kv heads: 2048 merges + 9 slots x 8 heads x 4 slices
    assert contracts.combine_grid(256, 8) == 2048 + 288
    # C2 and C3 (G 4): two-wave combine workgroups; C5 (G 8) four-wave ones
    assert f"grid {2048 + 288} x block 128" in contracts.render_workload("mi355x-rpa-c2")
    assert "rpa_combine_kernel: grid 2336 x block 256" in contracts.render_workload("mi355x-rpa-c5")
    assert re.search(r"int combine_waves\(const Params& p\) \{ return p\.G <= 4 && !p\.pf_kernel \? 2 : 4; \}",
                     KERNEL_SRC)
    assert [contracts.combine_waves(g) for g in (1, 2, 4, 8, 16)] == [2, 2, 2, 4, 4]


def test_mixed_plan_splits_prefill_and_decode():
    # C3 takes the co-resident layout: 4-wave workgroups, two per CU, tiles of 128 rows = 128 / G tokens
    text = contracts.render_workload("mi355x-rpa-c3")
    m = config_meta("c3")
    hkv, group = m.num_kv_heads, m.num_q_heads // m.num_kv_heads
    tq = 128 // group
    assert "co-resident>: grid 512 x block 256" in text
    tiles = sum(math.ceil(int(q) / tq) * hkv for q in m.q_lens if q >= 16)
    got = re.search(rf"prefill tiles = (\d+) tiles of {tq} tokens x 1 kv head \((\d+) chunk steps\); "
                    r"workgroups (\d+) \.\. (\d+) start on them", text)
    assert got and int(got.group(1)) == tiles
    # chunk steps of the causal tiles: tile t of a chunk sees prior + tq (t + 1) keys
    steps = sum(hkv * sum((int(L) - int(q) + tq * (t + 1)) / 32 for t in range(math.ceil(int(q) / tq)))
                for L, q in zip(m.kv_lens, m.q_lens) if q >= 16)
    assert int(got.group(2)) == round(steps)
    # at most one prefill-first workgroup per CU, numbered from grid / 2
    assert int(got.group(3)) == 256 and 256 <= int(got.group(4)) <= 511
    # merges (512 workgroups x 4 heads) + 17 heavy slots x 4 heads x 4 slices + 4 per CU for split tiles
    assert contracts.combine_grid(512, 4, co=True) == 2048 + 272 + 1024
    assert f"grid {2048 + 272 + 1024} x block 128" in text


def test_co_resident_gate_follows_resolve_layout():
    # resolve_layout's conditions, restated from the kernel source and checked against the model
    assert re.search(r"p\.S % KV_CHUNK == 0 && p\.Hkv % kCoWaves == 0 &&\s*p\.G <= 32 \* kCoWaves && "
                     r"\(long long\)shape->num_tokens >= \(long long\)shape->max_num_seqs \+ 15", KERNEL_SRC)
    assert re.search(r"constexpr int kCoWaves = 4;", KERNEL_SRC)
    assert contracts.co_resident(128, 8, 4, 64, 2048, 64, "bf16")
    assert contracts.co_resident(128, 8, 4, 32, 2048, 64, "fp8")
    assert not contracts.co_resident(128, 8, 4, 16, 2048, 64, "bf16")    # page not a multiple of 32
    assert not contracts.co_resident(128, 2, 4, 64, 2048, 64, "bf16")    # Hkv not a multiple of 4
    assert not contracts.co_resident(128, 8, 4, 64, 64 + 14, 64, "bf16")  # no room for a 16-token sequence
    assert not contracts.co_resident(64, 8, 4, 64, 2048, 64, "bf16")     # narrow heads run through stream-K
    for cfg in ("c2", "c4", "c5"):  # decode batches keep the 8-wave layout
        assert "co-resident" not in contracts.render_workload(f"mi355x-rpa-{cfg}")


def test_fused_plan_is_one_attention_launch():
    text = contracts.render_workload("mi355x-inkling-fused-rpa")
    assert "one call = the two launches below" in text
    assert "launch 0 = rpa_attn_kernel<KV_BF16_FUSED, page ids per key>: grid 1024 x block 128" in text
    # 1024 workgroups x 2 heads + 34 heavy slots x 2 heads x 4 slices + one per sequence (4)
    assert "launch 1 = rpa_combine_kernel: grid 2324 x block 128" in text
    assert "rpa_fused_prep_kernel" not in text and "launch 2" not in text


def test_cli_writes_artifacts(tmp_path, capsys):
    out = tmp_path / "exp.json"
    assert contracts.main(["experiment", "mi355x-inkling-rpa", "--output", str(out)]) == 0
    art = json.loads(out.read_text())
    assert f"id={art['experiment_id']}" in capsys.readouterr().out
    assert [t["name"] for t in art["workload"]["inputs"]] == [
        "query", "key_cache", "value_cache", "page_table", "sequence_lengths", "relative_bias"]
    plan = tmp_path / "plan.txt"
    assert contracts.main(["render-workload", "mi355x-inkling-rpa", "--output", str(plan)]) == 0
    assert hashlib.sha256(plan.read_bytes()).hexdigest() == art["schedule_sha256"]
    with pytest.raises(SystemExit):
        contracts.main(["experiment", "no-such-workload"])

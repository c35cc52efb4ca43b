"""Workload contracts for the RPA hot path on MI355X: ``render-workload`` and ``experiment``.

The reference describes each kernel workload by two artifacts (``src/tpu_cake/cli.py:655-676``):
``render-workload W`` prints the workload's schedule as canonical text, and ``experiment W`` prints
its ``KernelExperiment`` JSON (``src/tpu_cake/contracts.py:205-235``): the tensors, the numerical
contract, the target hardware, the benchmark protocol, the search policy, the profile
expectation, the sha256 of the rendered schedule, and an ``experiment_id`` that is the sha256 of
the rest of the JSON (sorted keys, compact separators).  Search and evidence code key their
results on those ids.

This module keeps that schema (the same field names, so a consumer of the reference's
artifacts reads these unchanged) for this build's workloads on one MI355X:

* ``inkling-rpa`` -- the reference's own row, reproduced exactly: its TPU7x schedule text
  (``examples/inkling-rpa.mlir``, written by ``tpu_cake_amd.schedule_text``) and its experiment
  (``contracts/inkling-rpa-experiment.json``);
* ``mi355x-inkling-rpa`` -- the v1 Inkling decode contract (``workloads/inkling_rpa.py:693-722``:
  B 4, H 4, D 32, separate K/V caches ``[32, 16, 4, 32]``, relative bias ``[4, 128]``) as executed
  here by ``tpu_cake_amd.inkling.inkling_rpa`` (C ABI ``rpa_inkling_decode``);
* ``mi355x-inkling-fused-rpa`` -- the v3 fused decode on the reference's fixture shapes
  (``workloads/inkling_rpa.py:413-468``), executed by ``tpu_cake_amd.fused`` (C ABI
  ``rpa_inkling_fused_decode``);
* ``mi355x-rpa-c1`` .. ``mi355x-rpa-c5`` -- the benchmark configurations of the operator
  ``ragged_paged_attention`` (C ABI ``rpa_ragged_paged_attention``).

The "schedule" of a workload here is its launch plan on MI355X: the kernels, grids and LDS, the
stream-K unit decomposition and its split into prefill tiles and stream-K pieces, and the
algorithmic bytes and FLOPs with the roofline floor they imply.  It is computed on the host from
the shapes (no GPU needed), with the work split restated from ``csrc/rpa_schedule.h`` and the
attention kernel's cost model.

Usage::

    python -m tpu_cake_amd list-workloads
    python -m tpu_cake_amd render-workload mi355x-rpa-c2 [--output PATH]
    python -m tpu_cake_amd experiment mi355x-rpa-c2 [--output PATH]
"""

from __future__ import annotations

import hashlib
import json
import math
import pathlib
from enum import Enum
from typing import Callable

from pydantic import BaseModel, ConfigDict, Field, computed_field, model_validator

from .cost_model import floors, mi355x_rates

PACKAGE = pathlib.Path(__file__).resolve().parent
ROOT = PACKAGE.parent.parent


class WorkloadStage(str, Enum):
    CONTROL = "control"
    PREFILL = "prefill"
    STEADY_DECODE = "steady_decode"
    MIXED = "mixed"


class ProfileExpectation(BaseModel):
    """What a captured profile must show.  On this target the "timed markers" are kernel names
    that must appear in the rocprofv3 kernel trace of the timed steps, the forbidden fragments
    are kernel-name fragments that must not (e.g. framework kernels in the timed region), and the
    HBM counters are rocprofv3 ``FETCH_SIZE`` / ``WRITE_SIZE``."""

    model_config = ConfigDict(extra="forbid", frozen=True)
    name: str = Field(min_length=1)
    stage: WorkloadStage
    minimum_tpu_device_planes: int = Field(default=1, ge=1)
    require_tensor_core_activity: bool = True
    require_hbm_read_counters: bool = False
    require_hbm_write_counters: bool = False
    require_cycle_counters: bool = False
    minimum_counter_device_planes: int = Field(default=0, ge=0)
    required_timed_hlo_markers: tuple[str, ...] = ()
    forbidden_timed_hlo_fragments: tuple[str, ...] = ()


class TargetHardware(BaseModel):
    """``vmem_budget_bytes_per_core`` is the LDS of one CU and ``smem_budget_bytes_per_core`` the
    scalar register file of one CU on this target."""

    model_config = ConfigDict(extra="forbid", frozen=True)
    accelerator: str = Field(min_length=1)
    topology: str = Field(min_length=1)
    chip_count: int = Field(ge=1)
    vmem_budget_bytes_per_core: int = Field(gt=0)
    smem_budget_bytes_per_core: int = Field(gt=0)
    peak_hbm_bytes_per_second: int | None = Field(default=None, gt=0)
    peak_flops_per_second: int | None = Field(default=None, gt=0)
    runtime_target: str = Field(min_length=1)


class TensorContract(BaseModel):
    model_config = ConfigDict(extra="forbid", frozen=True)
    name: str = Field(min_length=1)
    shape: tuple[int, ...]
    logical_shape: tuple[str, ...]
    dtype: str = Field(min_length=1)
    sharding: tuple[str, ...]

    @model_validator(mode="after")
    def ranks_match(self) -> "TensorContract":
        if len(self.shape) != len(self.logical_shape) or len(self.shape) != len(self.sharding):
            raise ValueError("tensor physical shape, logical shape, and sharding must have equal rank")
        if any(size <= 0 for size in self.shape):
            raise ValueError("tensor dimensions must be positive")
        return self


class NumericalContract(BaseModel):
    model_config = ConfigDict(extra="forbid", frozen=True)
    reference: str = Field(min_length=1)
    absolute_tolerance: float = Field(ge=0)
    relative_tolerance: float = Field(ge=0)
    deterministic: bool = True


class SourceFileContract(BaseModel):
    model_config = ConfigDict(extra="forbid", frozen=True)
    path: str = Field(min_length=1)
    sha256: str = Field(pattern=r"^[0-9a-f]{64}$")


class ExecutionContract(BaseModel):
    model_config = ConfigDict(extra="forbid", frozen=True)
    executor: str = Field(min_length=1)
    scope: str = Field(min_length=1)
    preflight: str | None = None
    source_revision: str | None = None
    source_manifest: tuple[SourceFileContract, ...] = ()

    @model_validator(mode="after")
    def source_paths_are_unique(self) -> "ExecutionContract":
        paths = [source.path for source in self.source_manifest]
        if len(paths) != len(set(paths)):
            raise ValueError("execution source manifest paths must be unique")
        return self


class BenchmarkProtocol(BaseModel):
    model_config = ConfigDict(extra="forbid", frozen=True)
    warmup_iterations: int = Field(ge=0)
    measured_iterations: int = Field(ge=1)
    synchronization: str = Field(min_length=1)
    statistic: str = Field(min_length=1)


class SearchPolicy(BaseModel):
    model_config = ConfigDict(extra="forbid", frozen=True)
    objective_metric: str = Field(min_length=1)
    require_correctness: bool = True
    require_profile_acceptance: bool = True


class WorkloadContract(BaseModel):
    model_config = ConfigDict(extra="forbid", frozen=True)
    name: str = Field(min_length=1)
    stage: WorkloadStage
    inputs: tuple[TensorContract, ...]
    outputs: tuple[TensorContract, ...]
    numerical: NumericalContract
    execution: ExecutionContract | None = None


class KernelExperiment(BaseModel):
    model_config = ConfigDict(extra="forbid", frozen=True)
    workload: WorkloadContract
    target: TargetHardware
    benchmark: BenchmarkProtocol
    search: SearchPolicy
    profile: ProfileExpectation
    schedule_sha256: str = Field(pattern=r"^[0-9a-f]{64}$")

    @computed_field
    @property
    def experiment_id(self) -> str:
        """sha256 of the experiment's JSON without this field (sorted keys, compact): the
        reference's id (src/tpu_cake/contracts.py:214-224)."""
        return _payload_id(_artifact_payload(self))


def _payload_id(payload: dict) -> str:
    return hashlib.sha256(json.dumps(payload, sort_keys=True, separators=(",", ":")).encode()).hexdigest()


def _artifact_payload(experiment: KernelExperiment, *, checked_in_form: bool = False) -> dict:
    """The fields an artifact carries: a workload without an execution contract omits it (the
    reference's rule, src/tpu_cake/contracts.py:219-222).  ``checked_in_form``: also omit the
    profile's ``minimum_counter_device_planes`` while it holds its default 0 -- the form of the
    reference's checked-in ``contracts/inkling-rpa-experiment.json``, written before that field
    existed (the reference's current code hashes the field, so its id for that row differs from
    the one the checked-in file carries)."""
    payload = experiment.model_dump(mode="json", exclude={"experiment_id"})
    if payload["workload"]["execution"] is None:
        del payload["workload"]["execution"]
    if checked_in_form and payload["profile"].get("minimum_counter_device_planes") == 0:
        del payload["profile"]["minimum_counter_device_planes"]
    return payload


def experiment_artifact_json(experiment: KernelExperiment, *, indent: int = 2, checked_in_form: bool = False) -> str:
    """The artifact: the experiment's fields and its id, indented.  ``checked_in_form``: the form of
    the reference's checked-in artifact, with the id computed over that form (see _artifact_payload)."""
    payload = _artifact_payload(experiment, checked_in_form=checked_in_form)
    return json.dumps(dict(payload, experiment_id=_payload_id(payload)), indent=indent)


def artifact_id(experiment: KernelExperiment, *, checked_in_form: bool = False) -> str:
    return _payload_id(_artifact_payload(experiment, checked_in_form=checked_in_form))


# ----------------------------------------------------------------------------------- target
_RATES = mi355x_rates()
MI355X_CUS = _RATES.compute_units
MI355X_LDS_PER_CU = _RATES.lds_bytes_per_cu
MI355X_SGPR_BYTES_PER_CU = 4 * 800 * 4      # 800 scalar registers per SIMD, four SIMDs
MI355X_HBM_BYTES_PER_S = _RATES.hbm_bytes_per_second
MI355X_BF16_FLOPS = _RATES.compute_flops_per_second
WAVES_PER_CU = 8                            # the attention kernel: 2 waves per SIMD
KV_CHUNK = 32                               # keys per stream-K unit (csrc/rpa_schedule.h)
ROW_BLOCK = 16
# LDS per wave of the attention kernel: the unit's V chunk (32 key rows x 288 B) and the K tile of the
# full-line path (32 key rows x 272 B) (csrc/rpa_kernels.hip, kVRow / kKtRow)
WAVE_LDS_BYTES = KV_CHUNK * (128 * 2 + 32) + KV_CHUNK * (128 * 2 + 16)
# split row blocks with this many contributors are merged by HEAVY_SLICES dim-slice workgroups per
# kv head, one helper slot per (HEAVY_CONTRIB - 1) workgroups (csrc/rpa_kernels.hip, kHeavyContrib)
HEAVY_CONTRIB = 32
HEAVY_SLICES = 4


def combine_waves(group: int) -> int:
    """Waves per combine workgroup (combine_waves in csrc/rpa_kernels.hip, default knobs): 2 when a
    decode row block's merge covers at most 4 rows (G <= 4), else 4."""
    return 2 if group <= 4 else 4


def combine_grid(grid: int, hg: int, co: bool = False, fused_seqs: int = 0) -> int:
    """Workgroups of one combine launch: (descriptor, kv head) merges, then the heavy-merge helpers,
    then (fused step) one per sequence storing its new token, or (co-resident layout) four per
    split-tile slot, one slot per CU."""
    return (grid * hg + ((grid - 1) // (HEAVY_CONTRIB - 1) + 1) * hg * HEAVY_SLICES + fused_seqs
            + (4 * MI355X_CUS if co else 0))
PF_MIN = 16                                 # query tokens that make a sequence a prefill one
PF_COST = 0.45                              # prefill chunk-step cost in stream-K units


def mi355x_target(topology: str = "one GPU") -> TargetHardware:
    return TargetHardware(
        accelerator="MI355X",
        topology=topology,
        chip_count=1,
        vmem_budget_bytes_per_core=MI355X_LDS_PER_CU,
        smem_budget_bytes_per_core=MI355X_SGPR_BYTES_PER_CU,
        peak_hbm_bytes_per_second=MI355X_HBM_BYTES_PER_S,
        peak_flops_per_second=MI355X_BF16_FLOPS,
        runtime_target="HIP gfx950 kernels in librpa.so through the C ABI of include/rpa.h",
    )


def _tensor(name: str, shape, logical, dtype: str) -> TensorContract:
    shape = tuple(int(x) for x in shape)
    return TensorContract(name=name, shape=shape, logical_shape=tuple(logical), dtype=dtype,
                          sharding=("",) * len(shape))


def _source_manifest() -> tuple[SourceFileContract, ...]:
    files = ("tpu-cake_amd/csrc/rpa_kernels.hip", "tpu-cake_amd/csrc/rpa_schedule.h", "include/rpa.h")
    return tuple(SourceFileContract(path=f, sha256=hashlib.sha256((ROOT / f).read_bytes()).hexdigest())
                 for f in files)


# -------------------------------------------------------------- the work split, on the host
def _heads_per_group(hkv: int) -> int:
    for g in range(min(hkv, 8), 1, -1):
        if hkv % g == 0:
            return g
    return 1


def _rb_units(kv_len: int, q_len: int, group: int, rb: int) -> int:
    """Units of row block rb: keys up to the causal limit of its last row (rpa_schedule.h)."""
    last_tok = min(q_len - 1, (rb * ROW_BLOCK + ROW_BLOCK - 1) // group)
    vis = min(kv_len - q_len + last_tok + 1, kv_len)
    return -(-vis // KV_CHUNK) if vis > 0 else 0


def _seq_units(kv_len: int, q_len: int, group: int) -> int:
    if q_len <= 0 or kv_len <= 0:
        return 0
    nrb = -(-(q_len * group) // ROW_BLOCK)
    return sum(_rb_units(kv_len, q_len, group, rb) for rb in range(nrb))


CO_WAVES = 4  # the co-resident layout's workgroups (csrc/rpa_kernels.hip, kCoWaves)


def co_resident(head_dim: int, hkv: int, group: int, page_size: int, num_tokens: int, max_num_seqs: int,
                kv_dtype: str) -> bool:
    """Whether a call takes the co-resident layout (resolve_layout with the default knobs): 128-dim
    heads, bf16 or fp8 KV, page size a multiple of 32, Hkv a multiple of 4, and a batch that can hold
    a sequence of 16 query tokens."""
    return (head_dim == 128 and kv_dtype in ("bf16", "fp8") and page_size % KV_CHUNK == 0
            and hkv % CO_WAVES == 0 and group <= 32 * CO_WAVES and num_tokens >= max_num_seqs + 15)


def _work_split(kv_lens, q_lens, hq: int, hkv: int, kv_dtype: str, prefill_tiles: bool, co: bool = False) -> dict:
    """Stream-K units, prefill tiles and the workgroup split the attention kernel computes; co: the
    co-resident layout (4-wave workgroups, two per CU, at most one prefill-first workgroup per CU)."""
    group = hq // hkv
    hg = CO_WAVES if co else _heads_per_group(hkv)
    ng = hkv // hg
    grid = MI355X_CUS * max(1, WAVES_PER_CU // hg)
    tiles_on = prefill_tiles and len(kv_lens) <= 256 and (co or (kv_dtype == "bf16" and hg == 8))
    pf_tq = 32 * hg // group if tiles_on else 0
    W, tiles, steps = 0, 0, 0.0
    for L, ql in zip(kv_lens, q_lens):
        L, ql = int(L), int(ql)
        if tiles_on and ql >= PF_MIN and L > 0:
            nt = -(-ql // pf_tq)
            tiles += nt * hkv
            steps += hkv * (nt * (L - ql) + pf_tq * 0.5 * nt * (nt + 1)) / KV_CHUNK
        else:
            W += _seq_units(L, ql, group) * ng
    gpre = 0
    if tiles:
        pw = PF_COST * steps
        gpre = max(1, int(grid * pw / (pw + W) + 0.5))
        if W > 0:
            gpre = min(gpre, grid - 1)
        if co:
            gpre = min(gpre, grid // 2)
        gpre = min(gpre, tiles)
    gd = grid - gpre
    return dict(group=group, heads_per_workgroup=hg, kv_head_groups=ng, grid=grid, stream_k_units=W,
                stream_k_workgroups=gd, units_per_workgroup=(W // gd, -(-W // gd)) if gd else (0, 0),
                prefill_tiles=tiles, prefill_tile_tokens=pf_tq, prefill_workgroups=gpre,
                prefill_chunk_steps=round(steps))


def _plan_text(name: str, lines: list[str]) -> str:
    return "\n".join([f"mi355x-rpa launch plan v1: {name}"] + lines) + "\n"


# --------------------------------------------------------------------------------- workloads
def _operator_workload(cfg: str) -> tuple[str, WorkloadContract, dict]:
    from .workloads import CONFIG_DESCRIPTIONS, config_meta

    m = config_meta(cfg)
    kvd = "f8e4m3" if m.kv_dtype == "fp8" else "bf16"
    inputs = [
        _tensor("q", (m.num_tokens, m.num_q_heads, m.head_dim), ("T", "Hq", "D"), "bf16"),
        _tensor("kv_pages", (m.pool_pages, m.page_size, 2 * m.num_kv_heads, m.head_dim), ("P", "S", "Hkv2", "D"), kvd),
        _tensor("kv_lens", (m.num_seqs,), ("N",), "i32"),
        _tensor("page_indices", (m.num_seqs, m.pages_per_seq), ("N", "PPS"), "i32"),
        _tensor("cu_q_lens", (m.num_seqs + 1,), ("N1",), "i32"),
        _tensor("num_seqs", (1,), ("One",), "i32"),
    ]
    if m.kv_dtype == "fp8":
        inputs.insert(2, _tensor("kv_scales", (m.pool_pages, m.num_kv_heads, 2), ("P", "Hkv", "KV"), "f32"))
    outputs = [_tensor("o", (m.num_tokens, m.num_q_heads, m.head_dim), ("T", "Hq", "D"), "bf16")]
    contract = WorkloadContract(
        name=f"ragged-paged-attention-{cfg}",
        stage=WorkloadStage.MIXED if int(max(m.q_lens)) > 1 else WorkloadStage.STEADY_DECODE,
        inputs=tuple(inputs), outputs=tuple(outputs),
        numerical=NumericalContract(reference="oracle.rpa_oracle.ref_ragged_paged_attention",
                                    absolute_tolerance=0.02, relative_tolerance=0.02),
        execution=ExecutionContract(executor="tpu_cake_amd.ops.ragged_paged_attention", scope="one GPU",
                                    preflight="tpu_cake_amd.ops.static_validate_inputs",
                                    source_manifest=_source_manifest()),
    )
    co = co_resident(m.head_dim, m.num_kv_heads, m.num_q_heads // m.num_kv_heads, m.page_size, m.num_tokens,
                     m.num_seqs, m.kv_dtype)
    split = _work_split(m.kv_lens, m.q_lens, m.num_q_heads, m.num_kv_heads, m.kv_dtype, prefill_tiles=True, co=co)
    work = m.work()
    kv_bytes = work.kv_read_bytes + work.scale_bytes
    qo_bytes = work.q_bytes + work.o_bytes
    flops = work.prefill_flops
    fl = floors(work, _RATES)
    hg = split["heads_per_workgroup"]
    unit_bytes = hg * KV_CHUNK * 2 * m.head_dim * (1 if m.kv_dtype == "fp8" else 2)
    mode = "KV_FP8" if m.kv_dtype == "fp8" else "KV_BF16"
    upg = m.page_size % KV_CHUNK == 0
    line = upg and m.kv_dtype != "fp8"
    floor_hbm = fl["hbm_s"] * 1e6
    floor_mfma = fl["mfma_s"] * 1e6
    half = split["grid"] // 2
    fixed = co and split["prefill_workgroups"] == half and half % 8 == 0
    lines = [
        f"description = {CONFIG_DESCRIPTIONS[cfg]}",
        "entry = rpa_ragged_paged_attention (include/rpa.h); one call = the two launches below, stream-ordered",
        f"sequences = {m.num_seqs}; query tokens = {m.num_tokens}; sum kv_len = {int(sum(m.kv_lens))}",
        f"heads = Hq {m.num_q_heads} / Hkv {m.num_kv_heads} (G {split['group']}); head_dim {m.head_dim}; "
        f"page_size {m.page_size}; pool pages {m.pool_pages}; pages per sequence {m.pages_per_seq}",
        f"launch 0 = rpa_attn_kernel<{mode}, page ids per {'chunk' if upg else 'key'}"
        f"{', co-resident' if co else ''}>: "
        f"grid {split['grid']} x block {64 * hg} ({hg} kv heads per workgroup, one wave each; "
        f"{WAVES_PER_CU} waves per CU), LDS {hg * WAVE_LDS_BYTES} B",
        f"  decode loads = {'whole 128-byte K/V lines, K through an LDS tile' if line else '16-byte operand loads'}",
        f"  stream-K = {split['stream_k_units']} units of {KV_CHUNK} keys x (sequence, kv-head group, "
        f"{ROW_BLOCK}-row block) over {split['stream_k_workgroups']} workgroups "
        f"({split['units_per_workgroup'][0]}..{split['units_per_workgroup'][1]} units each); "
        f"{unit_bytes} KV bytes per unit per workgroup",
    ]
    if co:
        lines.append(
            f"  prefill tiles = {split['prefill_tiles']} tiles of {split['prefill_tile_tokens']} tokens x 1 kv head "
            f"({split['prefill_chunk_steps']} chunk steps); workgroups {half} .. {half + split['prefill_workgroups'] - 1} "
            f"start on them, each beside the stream-K workgroup b - {half} on its CU, which joins when its range "
            f"is done; tiles queued per XCD (tile t on XCD t mod 8)"
            + (f", the first {2 * half // 8} positions of each XCD's queue fixed: the CU's prefill-first "
               f"workgroup position k, its stream-K workgroup {2 * half // 8 - 1} - k" if fixed else ""))
    else:
        lines.append(
            f"  prefill tiles = {split['prefill_tiles']} tiles of {split['prefill_tile_tokens']} tokens x 1 kv head "
            f"({split['prefill_chunk_steps']} chunk steps) on {split['prefill_workgroups']} workgroups")
    lines += [
        f"launch 1 = rpa_combine_kernel: grid {combine_grid(split['grid'], hg, co=co)} x block "
        f"{64 * combine_waves(split['group'])} (one workgroup per "
        f"(split descriptor, kv head), then {HEAVY_SLICES} per (heavy slot, kv head) for splits of "
        f">= {HEAVY_CONTRIB} workgroups" + (", then 4 per split-tile slot" if co else "") + ")",
        f"algorithmic = KV {kv_bytes} B + Q/O {qo_bytes} B + metadata {work.metadata_bytes} B; "
        f"QK/PV {work.flops} FLOP (prefill rows {flops})",
        f"roofline floor = HBM {floor_hbm:.2f} us; MFMA {floor_mfma:.2f} us; bound = {fl['bound']}",
    ]
    return _plan_text(f"mi355x-rpa-{cfg}", lines), contract, dict(kernels=("rpa_attn_kernel", "rpa_combine_kernel"))


def _inkling_v1_workload() -> tuple[str, WorkloadContract, dict]:
    B, H, D, P, S, MP, L = 4, 4, 32, 32, 16, 8, 128
    inputs = (
        _tensor("query", (B, H, D), ("B", "H", "D"), "bf16"),
        _tensor("key_cache", (P, S, H, D), ("P", "S", "H", "D"), "bf16"),
        _tensor("value_cache", (P, S, H, D), ("P", "S", "H", "D"), "bf16"),
        _tensor("page_table", (B, MP), ("B", "MP"), "i32"),
        _tensor("sequence_lengths", (B,), ("B",), "i32"),
        _tensor("relative_bias", (H, L), ("H", "L"), "bf16"),
    )
    outputs = (_tensor("output", (B, H, D), ("B", "H", "D"), "bf16"),)
    contract = WorkloadContract(
        name="inkling-ragged-paged-relative-bias-attention", stage=WorkloadStage.STEADY_DECODE,
        inputs=inputs, outputs=outputs,
        numerical=NumericalContract(reference="oracle.rpa_oracle.inkling_rpa_reference",
                                    absolute_tolerance=0.02, relative_tolerance=0.02),
        execution=ExecutionContract(executor="tpu_cake_amd.inkling.inkling_rpa", scope="one GPU",
                                    source_manifest=_source_manifest()),
    )
    split = _work_split([L] * B, [1] * B, H, H, "bf16", prefill_tiles=False)
    lines = [
        "description = v1 Inkling decode contract: separate K/V caches, additive relative bias [H, L] by key "
        "position, scale 1/D (workloads/inkling_rpa.py:37-73, :693-722)",
        "entry = rpa_inkling_decode (include/rpa.h); one call = the four launches below, stream-ordered",
        f"sequences = {B} (one query token each); heads = Hq {H} / Hkv {H}; head_dim {D} (rows padded to 128); "
        f"page_size {S}; pool pages {P}; pages per sequence {MP}",
        "launch 0 = rpa_inkling_v1_prep_kernel: grid-stride; packs the K/V caches into the combined "
        "[P, S, 2H, 128] layout, writes the bias table by key position, cu_q = 0..B, num_seqs, padded queries",
        f"launch 1 = rpa_attn_kernel<KV_BF16_BIAS>: grid {split['grid']} x block {64 * split['heads_per_workgroup']}; "
        f"at most {split['stream_k_units']} stream-K units (sequences up to {L} keys)",
        f"launch 2 = rpa_combine_kernel: grid {combine_grid(split['grid'], split['heads_per_workgroup'])} x block "
        f"{64 * combine_waves(split['group'])}",
        "launch 3 = rpa_fused_unpad_kernel: output rows 128 -> D",
    ]
    kernels = ("rpa_inkling_v1_prep_kernel", "rpa_attn_kernel", "rpa_combine_kernel", "rpa_fused_unpad_kernel")
    return _plan_text("mi355x-inkling-rpa", lines), contract, dict(kernels=kernels)


def _inkling_fused_workload() -> tuple[str, WorkloadContract, dict]:
    T, Hq, Hkv, D, P, S, R, E, N = 4, 4, 2, 32, 32, 16, 16, 128, 4
    inputs = (
        _tensor("queries", (T, Hq, D), ("T", "Hq", "D"), "bf16"),
        _tensor("keys", (T, Hkv, D), ("T", "Hkv", "D"), "bf16"),
        _tensor("values", (T, Hkv, D), ("T", "Hkv", "D"), "bf16"),
        _tensor("fused_cache", (P, S, Hkv, 2, 128), ("P", "S", "Hkv2p", "Pack", "Dpad"), "bf16"),
        _tensor("kv_lengths", (N,), ("N",), "i32"),
        _tensor("page_indices", (P,), ("PI",), "i32"),
        _tensor("cumulative_query_lengths", (N + 1,), ("N1",), "i32"),
        _tensor("cumulative_kv_lengths", (N + 1,), ("N1",), "i32"),
        _tensor("distribution", (3,), ("R3",), "i32"),
        _tensor("relative_states", (T, Hq, R), ("T", "Hq", "R"), "bf16"),
        _tensor("relative_projection", (R, E), ("R", "E"), "bf16"),
    )
    outputs = (
        _tensor("output", (T, Hq, D), ("T", "Hq", "D"), "bf16"),
        _tensor("updated_fused_cache", (P, S, Hkv, 2, 128), ("P", "S", "Hkv2p", "Pack", "Dpad"), "bf16"),
    )
    contract = WorkloadContract(
        name="inkling-fused-ragged-paged-relative-bias-decode", stage=WorkloadStage.STEADY_DECODE,
        inputs=inputs, outputs=outputs,
        numerical=NumericalContract(reference="oracle.rpa_fused_oracle.inkling_fused_rpa_reference",
                                    absolute_tolerance=0.02, relative_tolerance=0.02),
        execution=ExecutionContract(executor="tpu_cake_amd.fused.invoke", scope="one GPU",
                                    preflight="tpu_cake_amd.fused.preflight", source_manifest=_source_manifest()),
    )
    split = _work_split([S * MP for MP in (1, 2, 3, 4)], [1] * N, Hq, Hkv, "bf16", prefill_tiles=False)
    lines = [
        "description = v3 fused Inkling decode: new K/V rows written into the paged cache at kv_len - 1, "
        "relative-position bias relative_states . relative_projection for distances < E, scale 1/D "
        "(workloads/inkling_rpa.py:471-589)",
        "entry = rpa_inkling_fused_decode (include/rpa.h), after the host preflight "
        "(rpa_lowering.py:71-128); one call = the two launches below, stream-ordered",
        f"tokens = sequences = {N}; heads = Hq {Hq} / Hkv {Hkv}; head_dim {D} (cache rows padded to 128); "
        f"page_size {S}; pages {P}; relative states R {R}, extent E {E}",
        f"launch 0 = rpa_attn_kernel<KV_BF16_FUSED, page ids per key>: grid {split['grid']} x block "
        f"{64 * split['heads_per_workgroup']}; sequence i's pages from page_indices[cu_kv_lens[i] / S], its new "
        "token's K/V read from keys/values, queries and output rows D wide, the relative bias formed in the "
        "kernel (one 16x16x16 MFMA per 16 keys)",
        f"launch 1 = rpa_combine_kernel: grid {combine_grid(split['grid'], split['heads_per_workgroup'], fused_seqs=N)}"
        f" x block {64 * combine_waves(split['group'])}; the last N workgroups store each sequence's new K/V rows "
        "in its cache slot",
    ]
    kernels = ("rpa_attn_kernel", "rpa_combine_kernel")
    return _plan_text("mi355x-inkling-fused-rpa", lines), contract, dict(kernels=kernels)


# ----------------------------------------------------------------- the reference's own row
def _reference_inkling_rpa() -> tuple[str, KernelExperiment]:
    """``render-workload`` / ``experiment inkling-rpa`` as the reference prints them: its TPU7x
    schedule text and ``KernelExperiment`` (``inkling_rpa_contract`` / ``inkling_rpa_experiment``,
    src/tpu_cake/workloads/inkling_rpa.py:693-722, :937-964), reproducing
    ``examples/inkling-rpa.mlir`` and ``contracts/inkling-rpa-experiment.json`` byte for byte."""
    from .schedule_text import inkling_rpa_schedule_text

    def t(name, shape, logical):
        return _tensor(name, shape, logical.split(), "i32" if name in ("page_table", "sequence_lengths") else "bf16")

    text = inkling_rpa_schedule_text()
    workload = WorkloadContract(
        name="inkling-ragged-paged-relative-bias-attention", stage=WorkloadStage.STEADY_DECODE,
        inputs=(t("query", (4, 4, 32), "B H D"), t("key_cache", (32, 16, 4, 32), "P S H D"),
                t("value_cache", (32, 16, 4, 32), "P S H D"), t("page_table", (4, 8), "B MP"),
                t("sequence_lengths", (4,), "B"), t("relative_bias", (4, 128), "H L")),
        outputs=(t("output", (4, 4, 32), "B H D"),),
        numerical=NumericalContract(reference="tpu_cake.workloads.inkling_rpa.inkling_rpa_reference",
                                    absolute_tolerance=0.02, relative_tolerance=0.02),
    )
    exp = KernelExperiment(
        workload=workload,
        target=TargetHardware(accelerator="TPU7x", topology="4x1", chip_count=4, vmem_budget_bytes_per_core=2 << 20,
                              smem_budget_bytes_per_core=1 << 16, runtime_target="Pallas Mosaic TPU"),
        benchmark=BenchmarkProtocol(warmup_iterations=5, measured_iterations=50,
                                    synchronization="block until device result is ready",
                                    statistic="median device duration"),
        search=SearchPolicy(objective_metric="median_device_duration_ns"),
        profile=ProfileExpectation(name="inkling-rpa-steady-decode", stage=WorkloadStage.STEADY_DECODE,
                                   minimum_tpu_device_planes=8, required_timed_hlo_markers=("ragged_paged_attention",),
                                   forbidden_timed_hlo_fragments=("12582912,16", "native_backend.py:500")),
        schedule_sha256=hashlib.sha256(text.encode()).hexdigest(),
    )
    return text, exp


# the reference's rows (its CLI's _WORKLOADS, src/tpu_cake/cli.py:148-151, RPA part)
REFERENCE_WORKLOADS = {"inkling-rpa": _reference_inkling_rpa}

# this build's rows: the MI355X launch plans
WORKLOADS: dict[str, Callable[[], tuple[str, WorkloadContract, dict]]] = {
    "mi355x-inkling-rpa": _inkling_v1_workload,
    "mi355x-inkling-fused-rpa": _inkling_fused_workload,
    **{f"mi355x-rpa-c{i}": (lambda c=f"c{i}": _operator_workload(c)) for i in range(1, 6)},
}
ALL_WORKLOADS = (*REFERENCE_WORKLOADS, *WORKLOADS)


def render_workload(name: str) -> str:
    """The workload's schedule: the reference's TPU schedule text for its own rows, the launch plan
    on MI355X for this build's (canonical text; its sha256 is the experiment's ``schedule_sha256``)."""
    if name in REFERENCE_WORKLOADS:
        return REFERENCE_WORKLOADS[name]()[0]
    if name not in WORKLOADS:
        raise ValueError(f"unknown workload {name!r}; expected one of {sorted(ALL_WORKLOADS)}")
    return WORKLOADS[name]()[0]


def experiment(name: str) -> KernelExperiment:
    if name in REFERENCE_WORKLOADS:
        return REFERENCE_WORKLOADS[name]()[1]
    if name not in WORKLOADS:
        raise ValueError(f"unknown workload {name!r}; expected one of {sorted(ALL_WORKLOADS)}")
    text, contract, extra = WORKLOADS[name]()
    return KernelExperiment(
        workload=contract,
        target=mi355x_target(),
        benchmark=BenchmarkProtocol(
            warmup_iterations=5, measured_iterations=50,
            synchronization="hipEventSynchronize on timing-only events recorded around the call's kernels",
            statistic="median device duration",
        ),
        search=SearchPolicy(objective_metric="median_device_duration_ns"),
        profile=ProfileExpectation(
            name=f"{name}-{contract.stage.value}", stage=contract.stage, minimum_tpu_device_planes=1,
            require_tensor_core_activity=True, require_hbm_read_counters=True, require_hbm_write_counters=True,
            required_timed_hlo_markers=extra["kernels"],
            forbidden_timed_hlo_fragments=("at::native", "__amd_rocclr_copyBuffer"),
        ),
        schedule_sha256=hashlib.sha256(text.encode()).hexdigest(),
    )


def main(argv=None) -> int:
    import argparse

    ap = argparse.ArgumentParser(prog="python -m tpu_cake_amd",
                                 description="Workload contracts of the RPA hot path on MI355X")
    sub = ap.add_subparsers(dest="cmd", required=True)
    sub.add_parser("list-workloads")
    for cmd in ("render-workload", "experiment"):
        sp = sub.add_parser(cmd)
        sp.add_argument("workload", choices=sorted(ALL_WORKLOADS))
        sp.add_argument("--output", type=pathlib.Path)
        if cmd == "experiment":
            sp.add_argument("--checked-in-form", action="store_true",
                            help="write the form of the reference's checked-in artifacts (no "
                                 "minimum_counter_device_planes while it is 0), id over that form")
    args = ap.parse_args(argv)
    if args.cmd == "list-workloads":
        for name in ALL_WORKLOADS:
            print(name)
        return 0
    if args.cmd == "render-workload":
        rendered = render_workload(args.workload)
        if args.output is None:
            print(rendered, end="")
        else:
            args.output.parent.mkdir(parents=True, exist_ok=True)
            args.output.write_text(rendered)
            print(f"WORKLOAD_RENDERED workload={args.workload} path={args.output}")
        return 0
    exp = experiment(args.workload)
    rendered = experiment_artifact_json(exp, checked_in_form=args.checked_in_form) + "\n"
    if args.output is None:
        print(rendered, end="")
    else:
        args.output.parent.mkdir(parents=True, exist_ok=True)
        args.output.write_text(rendered)
        print(f"EXPERIMENT_WRITTEN workload={args.workload} id={artifact_id(exp, checked_in_form=args.checked_in_form)} "
              f"path={args.output}")
    return 0

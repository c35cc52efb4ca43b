"""MI355X rates and the RPA work convention: the algorithmic bytes and FLOPs of one call.

The reference prices schedules with a ``HardwareRateModel`` of sourced rates
(``src/tpu_cake/cost_model.py:20-31``; ``tpu7x_tensorcore_rates``, :95-106) and its physical cost
model refuses RPA ops for want of a work convention (``physical_cost_model.py:800-812``: "has no
work convention for ...ragged_paged_attention").  This module is both for this build:

* ``mi355x_rates()`` -- the same model with MI355X's published rates and where each comes from
  (and, when measured, the copy probe's achieved HBM bandwidth as the practical ceiling);
* ``rpa_work(...)`` -- the work convention of one ``ragged_paged_attention`` call: the KV bytes it
  must read (each key a row of the sequence's causal window reads once: K and V of every kv head),
  query/output/metadata/scale bytes, and the QK^T + PV FLOPs of every (row, visible key);
* ``floors(work, rates)`` -- the roofline floor each resource implies and the binding one.

``bench.py``, the launch plans of ``tpu_cake_amd.contracts`` and the cases of
``tpu_cake_amd.workloads`` all count with ``rpa_work``.
"""

from __future__ import annotations

import dataclasses

import numpy as np
from pydantic import BaseModel, ConfigDict, Field


class HardwareRateModel(BaseModel):
    """Rates of one device, each with a status note saying where it comes from (the reference's
    model, with MI355X's xGMI link in the interconnect field and the fp8 peak and on-chip sizes
    the RPA kernels need)."""

    model_config = ConfigDict(extra="forbid", frozen=True)

    name: str = Field(min_length=1)
    scope: str = Field(min_length=1)
    compute_flops_per_second: int = Field(gt=0)      # dense bf16 MFMA
    fp8_flops_per_second: int = Field(gt=0)          # dense fp8 MFMA
    hbm_bytes_per_second: int = Field(gt=0)
    ici_bytes_per_second: int = Field(gt=0)          # one xGMI link, one direction
    compute_units: int = Field(gt=0)
    lds_bytes_per_cu: int = Field(gt=0)
    last_level_cache_bytes: int = Field(gt=0)        # Infinity Cache (MALL)
    compute_status: str = Field(min_length=1)
    hbm_status: str = Field(min_length=1)
    ici_status: str = Field(min_length=1)
    source_url: str = Field(min_length=1)
    measured_hbm_bytes_per_second: int | None = Field(default=None, gt=0)
    measured_status: str | None = None


def mi355x_rates(measured_copy_bytes_per_second: float | None = None) -> HardwareRateModel:
    """MI355X (gfx950) published peaks.  ``measured_copy_bytes_per_second``: a device-to-device copy's
    achieved (read + write) bandwidth on the box, recorded beside the peak."""
    return HardwareRateModel(
        name="MI355X",
        scope="one GPU (8 XCDs, 256 compute units)",
        compute_flops_per_second=2_500_000_000_000_000,
        fp8_flops_per_second=5_000_000_000_000_000,
        hbm_bytes_per_second=8_000_000_000_000,
        ici_bytes_per_second=153_600_000_000,
        compute_units=256,
        lds_bytes_per_cu=160 * 1024,
        last_level_cache_bytes=256 * 1024 * 1024,
        compute_status="AMD published dense MFMA peaks (bf16 2.5 PFLOP/s, fp8 5.0 PFLOP/s; the sparse "
                       "figures are twice these and not used)",
        hbm_status="AMD published HBM3E peak, 8 TB/s over 288 GB",
        ici_status="AMD published xGMI: 7 links per GPU at about 153.6 GB/s each (not used: one GPU)",
        source_url="https://www.amd.com/en/products/accelerators/instinct/mi350/mi355x.html",
        measured_hbm_bytes_per_second=int(measured_copy_bytes_per_second) if measured_copy_bytes_per_second else None,
        measured_status=("device-to-device copy on the box (bench.py --copy-probe): bytes read + written / time"
                         if measured_copy_bytes_per_second else None),
    )


@dataclasses.dataclass(frozen=True)
class RpaWork:
    """Algorithmic work of one call (no re-reads, no padding)."""
    kv_read_bytes: int        # K and V rows of every key some row of its sequence sees, every kv head
    scale_bytes: int          # fp8 per-(page, kv head) K and V scales of the pages read
    q_bytes: int
    o_bytes: int
    metadata_bytes: int       # kv_lens, cu_q_lens, the page ids of the pages read, num_seqs
    flops: int                # QK^T + PV: 4 * D per (query head row, visible key)
    prefill_flops: int        # the part of ``flops`` in sequences with more than one query token
    visible_keys: int         # sum over (query token, q head) rows of their visible keys / Hq
    keys_read: int            # sum over sequences of the keys read

    @property
    def hbm_bytes(self) -> int:
        return self.kv_read_bytes + self.scale_bytes + self.q_bytes + self.o_bytes + self.metadata_bytes


def _keys(kv_len: int, q_len: int, window: int | None) -> tuple[int, int]:
    """(keys read, sum over the sequence's query tokens of visible keys): token j sits at position
    p = kv_len - q_len + j and sees keys (p - window, p] (all of [0, p] without a window)."""
    if kv_len <= 0 or q_len <= 0:
        return 0, 0
    pos = kv_len - q_len + np.arange(q_len, dtype=np.int64)
    pos = pos[pos >= 0]
    if pos.size == 0:
        return 0, 0
    hi = pos + 1
    lo = np.zeros_like(pos) if not window else np.maximum(pos - window + 1, 0)
    read = int(hi[-1] - lo[0])
    return read, int(np.sum(hi - lo))


def rpa_work(kv_lens, q_lens, *, num_q_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
             kv_dtype: str = "bf16", sliding_window: int | None = None) -> RpaWork:
    """The work convention of ``ragged_paged_attention`` over sequences ``kv_lens`` / ``q_lens``
    (the causal rule of ragged_paged_attention.py:134-138 and its window, :532-534)."""
    if kv_dtype not in ("bf16", "fp8"):
        raise ValueError(f"kv_dtype must be 'bf16' or 'fp8', got {kv_dtype!r}")
    elem = 1 if kv_dtype == "fp8" else 2
    kv_lens = [int(x) for x in kv_lens]
    q_lens = [int(x) for x in q_lens]
    if len(kv_lens) != len(q_lens):
        raise ValueError("kv_lens and q_lens must have one entry per sequence")
    keys_read = vis = vis_pf = pages = 0
    for L, ql in zip(kv_lens, q_lens):
        r, v = _keys(L, ql, sliding_window)
        keys_read += r
        vis += v
        if ql > 1:
            vis_pf += v
        if r:
            lo = L - r
            pages += (L - 1) // page_size - lo // page_size + 1
    T = sum(q_lens)
    row = num_kv_heads * 2 * head_dim * elem
    return RpaWork(
        kv_read_bytes=keys_read * row,
        scale_bytes=pages * num_kv_heads * 2 * 4 if kv_dtype == "fp8" else 0,
        q_bytes=T * num_q_heads * head_dim * 2,
        o_bytes=T * num_q_heads * head_dim * 2,
        metadata_bytes=4 * (2 * len(kv_lens) + 2 + pages),
        flops=4 * num_q_heads * head_dim * vis,
        prefill_flops=4 * num_q_heads * head_dim * vis_pf,
        visible_keys=vis,
        keys_read=keys_read,
    )


def floors(work: RpaWork, rates: HardwareRateModel | None = None, *, kv_dtype: str = "bf16") -> dict:
    """Roofline floors (seconds) of a call: HBM bytes at the HBM peak, MFMA FLOPs at the bf16 peak
    (the kernels run both products in bf16, fp8 KV included); ``bound`` names the larger."""
    rates = rates or mi355x_rates()
    hbm = work.hbm_bytes / rates.hbm_bytes_per_second
    mfma = work.flops / rates.compute_flops_per_second
    return {"hbm_s": hbm, "mfma_s": mfma, "bound": "mfma" if mfma > hbm else "hbm", "floor_s": max(hbm, mfma)}

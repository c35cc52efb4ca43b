"""The RPA work convention and MI355X rates (tpu_cake_amd.cost_model) on the CPU: bytes and FLOPs
against a brute-force count over (query row, key) pairs with the reference's causal and window
masks (ragged_paged_attention.py:134-138, :532-534), and the published rates."""

import numpy as np
import pytest

from tpu_cake_amd import cost_model
from tpu_cake_amd.workloads import config_meta, make_custom


def _brute(kv_lens, q_lens, hq, hkv, d, page, elem, window):
    keys_read = vis = vis_pf = pages = 0
    for L, ql in zip(kv_lens, q_lens):
        seen = set()
        for j in range(ql):
            pos = L - ql + j
            for k in range(L):
                masked = k > pos or (window is not None and pos - window >= k)
                if not masked:
                    seen.add(k)
                    vis += 1
                    vis_pf += ql > 1
        keys_read += len(seen)
        pages += len({k // page for k in seen})
    return dict(kv=keys_read * hkv * 2 * d * elem, flops=4 * hq * d * vis, pf=4 * hq * d * vis_pf, pages=pages)


@pytest.mark.parametrize("window", [None, 1, 7, 40, 1000])
@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
def test_work_matches_brute_force(window, dtype):
    kv, ql = [1, 17, 64, 130, 5, 90], [1, 1, 64, 33, 0, 7]
    w = cost_model.rpa_work(kv, ql, num_q_heads=8, num_kv_heads=2, head_dim=16, page_size=16, kv_dtype=dtype,
                            sliding_window=window)
    b = _brute(kv, ql, 8, 2, 16, 16, 1 if dtype == "fp8" else 2, window)
    assert w.kv_read_bytes == b["kv"] and w.flops == b["flops"] and w.prefill_flops == b["pf"]
    assert w.scale_bytes == (b["pages"] * 2 * 2 * 4 if dtype == "fp8" else 0)
    assert w.q_bytes == w.o_bytes == sum(ql) * 8 * 16 * 2


def test_decode_kv_bytes_are_sum_of_lengths_times_row():
    m = config_meta("c2")
    w = m.work()
    assert w.kv_read_bytes == int(m.kv_lens.sum()) * 8 * 2 * 128 * 2  # sum(L) * 4 KiB
    assert w.prefill_flops == 0 and w.flops == 4 * 32 * 128 * int(m.kv_lens.sum())
    # a 512-key window reads min(L, 512) keys per decode row
    w512 = m.work(sliding_window=512)
    assert w512.kv_read_bytes == int(np.minimum(m.kv_lens, 512).sum()) * 4096


def test_case_and_meta_agree():
    case = make_custom(kv_lens=[300, 45, 1030], q_lens=[1, 45, 130], num_q_heads=32, num_kv_heads=8,
                       page_size=64, seed=3, values="host")
    w = case.work()
    assert case.kv_read_bytes() == w.kv_read_bytes and case.prefill_flops() == w.prefill_flops
    assert w.prefill_flops == 4 * 32 * 128 * (sum(range(1, 46)) + sum(900 + j + 1 for j in range(130)))


def test_rates_and_floors():
    r = cost_model.mi355x_rates()
    assert r.hbm_bytes_per_second == 8_000_000_000_000 and r.compute_flops_per_second == 2_500_000_000_000_000
    assert r.fp8_flops_per_second == 2 * r.compute_flops_per_second and r.compute_units == 256
    assert r.measured_hbm_bytes_per_second is None
    assert cost_model.mi355x_rates(6.1e12).measured_hbm_bytes_per_second == 6_100_000_000_000
    w = config_meta("c3").work()
    f = cost_model.floors(w, r)
    assert f["hbm_s"] == pytest.approx(w.hbm_bytes / 8e12) and f["mfma_s"] == pytest.approx(w.flops / 2.5e15)
    assert f["bound"] == "hbm" and f["floor_s"] == f["hbm_s"]

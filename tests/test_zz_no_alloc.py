"""The allocation-free entry point (rpa_ragged_paged_attention_noalloc, workspace in a file-scope
device array) against the operator's entry point with a caller workspace, through the C ABI: two
calls in a row, the second with a smaller input, each bitwise equal to the workspace entry's
output (same kernels, same persistent grid, same partition)."""

import ctypes
import sys

import numpy as np
import pytest
import torch

from oracle import rpa_oracle as orc
from tpu_cake_amd import _lib, ops
from tpu_cake_amd.workloads import make_custom

pytestmark = pytest.mark.gpu


def _noalloc(d, case, **knobs):
    plan_knobs = dict(sm_scale=case.sm_scale, sliding_window=None, soft_cap=None, mask_value=ops.DEFAULT_MASK_VALUE,
                      k_scale=None, v_scale=None, num_kv_pages_per_block=None, num_queries_per_block=None,
                      vmem_limit_bytes=None, waves_per_cu=None, prefill_tiles=None, prefill_cost=None)
    plan_knobs.update(knobs)
    kv_scales = d.get("kv_scales")
    shape, opts = ops._static_plan(d["q"], d["kv_pages"], d["kv_lens"], d["page_indices"], d["cu_q_lens"],
                                   d["num_seqs"], kv_scales, plan_knobs)
    out = torch.full_like(d["q"], 7.0)  # stale values: every row must be written
    stream = torch.cuda.current_stream().cuda_stream
    rc = _lib.load().rpa_ragged_paged_attention_noalloc(
        ctypes.byref(shape), ctypes.byref(opts), d["q"].data_ptr(), d["kv_pages"].data_ptr(),
        kv_scales.data_ptr() if kv_scales is not None else None, d["kv_lens"].data_ptr(),
        d["page_indices"].data_ptr(), d["cu_q_lens"].data_ptr(), d["num_seqs"].data_ptr(), out.data_ptr(), stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _with_workspace(d, case, **knobs):
    out = ops.ragged_paged_attention(d["q"], d["kv_pages"], d["kv_lens"], d["page_indices"], d["cu_q_lens"],
                                     d["num_seqs"], sm_scale=case.sm_scale, kv_scales=d.get("kv_scales"), **knobs)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


CASES = [
    # (kv_lens, q_lens, hq, hkv, page, kv_dtype): decode with long split sequences (heavy merges), then
    # a smaller batch with a prefill chunk (the tile queue), then a small fp8 one
    ([9000, 3000, 40, 7000, 2500, 64] * 6, [1] * 36, 32, 8, 64, "bf16"),
    ([700, 45, 1030, 9], [1, 45, 130, 1], 32, 8, 64, "bf16"),
    ([300, 5, 77], [1, 1, 3], 16, 4, 16, "fp8"),
]


def test_noalloc_matches_the_workspace_entry_on_consecutive_calls(cuda):
    for i, (kv, ql, hq, hkv, page, dt) in enumerate(CASES):
        print(f"[case] noalloc call {i}: {len(kv)} seqs, hq {hq} hkv {hkv} page {page} {dt}", flush=True)
        case = make_custom(kv_lens=kv, q_lens=ql, num_q_heads=hq, num_kv_heads=hkv, page_size=page, seed=300 + i,
                           kv_dtype=dt)
        d = ops.case_to_device(case, "cuda")
        got = _noalloc(d, case)
        want = _with_workspace(d, case)
        assert np.array_equal(got, want), f"call {i}: max diff {np.abs(got - want).max()}"
        ref = orc.bf16_round(orc.ref_ragged_paged_attention(
            case.q, case.kv_pages, case.kv_lens, case.page_indices, case.cu_q_lens, case.num_seqs,
            sm_scale=case.sm_scale, kv_scales=case.kv_scales, kv_dtype=case.kv_dtype))
        assert orc.errors(got[: ref.shape[0]], ref)["max_abs"] <= 2e-2
        # again right away, so this call reads the descriptors and flags the last one left
        assert np.array_equal(_noalloc(d, case), want)


def test_noalloc_knobs_and_window(cuda):
    print("[case] noalloc with knobs and a window", flush=True)
    case = make_custom(kv_lens=[5000, 300, 2000], q_lens=[1, 64, 1], num_q_heads=32, num_kv_heads=8, page_size=64,
                       seed=310)
    d = ops.case_to_device(case, "cuda")
    for kw in (dict(waves_per_cu=3), dict(sliding_window=200), dict(prefill_tiles=False)):
        assert np.array_equal(_noalloc(d, case, **kw), _with_workspace(d, case, **kw)), kw


def test_noalloc_rejects_bad_arguments_before_any_launch(cuda):
    lib = _lib.load()
    shape = _lib.RpaShape(4, 8, 2, 192, 10, 16, 4, 4, 0)  # a head dim that is not built
    rc = lib.rpa_ragged_paged_attention_noalloc(ctypes.byref(shape), ctypes.byref(_lib.RpaOptions(sm_scale=1.0)),
                                                *([None] * 8), None)
    assert rc == -2 and b"head_dim" in lib.rpa_last_error()
    rc = lib.rpa_ragged_paged_attention_noalloc(ctypes.byref(_lib.RpaShape(4, 8, 2, 128, 10, 16, 4, 4, 0)), None,
                                                *([None] * 8), None)
    assert rc == -1 and b"options" in lib.rpa_last_error()

"""GPU parity at the edges: every schedule-knob value the search may try or promote, sliding-window
chunk skipping, negative soft caps, out-of-range page ids, GQA groups that are not powers of two,
and one sequence at the longest C5 length (131072 keys).

Bar: max-abs <= 2e-2 against the oracle on the same inputs (bf16 output, fp32 accumulation), as in
test_gpu_parity; knob variants must also agree with each other to that bar.  Every case prints its
name first so a failing GPU step names it.
"""

import sys

import numpy as np
import pytest
import torch

from oracle import rpa_oracle as orc
from tpu_cake_amd import ops
from tpu_cake_amd.workloads import make_config, make_custom

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _ref(case, **kw):
    return orc.bf16_round(orc.ref_ragged_paged_attention(
        case.q, case.kv_pages, case.kv_lens, case.page_indices, case.cu_q_lens, case.num_seqs,
        sm_scale=case.sm_scale, kv_scales=case.kv_scales, kv_dtype=case.kv_dtype, **kw))


def _run(d, case, **kw):
    kv_scales = d.get("kv_scales")
    out = ops.ragged_paged_attention(d["q"], d["kv_pages"], d["kv_lens"], d["page_indices"], d["cu_q_lens"],
                                     d["num_seqs"], sm_scale=case.sm_scale, kv_scales=kv_scales, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _assert_close(got, ref, what):
    err = orc.errors(got[: ref.shape[0]], ref)
    print(f"  {what}: max_abs={err['max_abs']:.3e}", flush=True)
    assert err["finite"] and err["max_abs"] <= TOL, (what, err)


# ------------------------------------------------------------------------------------- knobs
@pytest.fixture(scope="module")
def c3_case():
    case = make_config("c3")
    return case, ops.case_to_device(case, "cuda"), _ref(case)


@pytest.fixture(scope="module")
def c5_case():
    case = make_config("c5")
    return case, ops.case_to_device(case, "cuda"), _ref(case)


@pytest.mark.parametrize("wpc", [1, 2, 3, 4, 5, 6, 7, 8])
def test_waves_per_cu_on_c3_and_c5(cuda, c3_case, c5_case, wpc):
    for name, (case, d, ref) in (("c3", c3_case), ("c5", c5_case)):
        _say(f"{name} waves_per_cu={wpc}")
        _assert_close(_run(d, case, waves_per_cu=wpc), ref, f"{name} waves_per_cu={wpc}")


@pytest.mark.parametrize("cost", [0.35, 0.45, 0.5, 0.6, 0.7])
def test_prefill_cost_on_c3(cuda, c3_case, cost):
    case, d, ref = c3_case
    _say(f"c3 prefill_cost={cost}")
    _assert_close(_run(d, case, prefill_cost=cost), ref, f"prefill_cost={cost}")


@pytest.mark.parametrize("wpc", [0, 3])
def test_prefill_tiles_off_on_c3(cuda, c3_case, wpc):
    case, d, ref = c3_case
    _say(f"c3 prefill tiles off, waves_per_cu={wpc}")
    _assert_close(_run(d, case, prefill_tiles=False, waves_per_cu=wpc), ref, "prefill tiles off")


def test_tuned_table_entry_matches_explicit_knobs(cuda, c3_case):
    """The wrapper's tuned-table lookup (no knobs given) runs exactly what the entry says."""
    from tpu_cake_amd import tuned

    case, d, ref = c3_case
    _say("c3 tuned table lookup")
    knobs = tuned.get_tuned_knobs("bf16", 4, 64, int(case.cu_q_lens[-1]))
    a = _run(d, case)
    b = _run(d, case, **knobs)
    assert np.array_equal(a, b)
    _assert_close(a, ref, "tuned")


# ------------------------------------------------------------------------------------- window
@pytest.mark.parametrize("window,page,kv_dtype", [(512, 64, "bf16"), (100, 16, "bf16"), (33, 64, "fp8"),
                                                  (512, 24, "bf16"), (4096, 64, "bf16")])
def test_sliding_window_skips_chunks_in_decode(cuda, window, page, kv_dtype):
    """Long decode rows with a window: the stream-K units start at the window's first chunk."""
    _say(f"decode window={window} page={page} {kv_dtype}")
    lens = [8000, 513, 2048, 31, 5000, 700, 6100, 1]
    case = make_custom(kv_lens=lens, q_lens=[1] * len(lens), num_q_heads=32, num_kv_heads=8, page_size=page,
                       seed=window + page, kv_dtype=kv_dtype)
    d = ops.case_to_device(case, "cuda")
    _assert_close(_run(d, case, sliding_window=window), _ref(case, sliding_window=window), "window")


@pytest.mark.parametrize("tiles", [True, False])
def test_sliding_window_with_query_chunks(cuda, tiles):
    """Chunked prefill rows with a window, through the prefill tiles and through stream-K row blocks
    (each row block starts at its own first row's window)."""
    _say(f"chunked prefill + window, prefill_tiles={tiles}")
    case = make_custom(kv_lens=[3000, 900, 1500, 64], q_lens=[200, 1, 333, 64], num_q_heads=32, num_kv_heads=8,
                       page_size=64, seed=91)
    d = ops.case_to_device(case, "cuda")
    _assert_close(_run(d, case, sliding_window=300, prefill_tiles=tiles), _ref(case, sliding_window=300), "window")


def test_sliding_window_with_finite_mask_value_visits_every_key(cuda):
    """With a finite mask value masked keys keep weight exp(s + mask - m), so no chunk is skipped."""
    _say("window + finite mask value")
    case = make_custom(kv_lens=[3000, 200], q_lens=[1, 5], num_q_heads=16, num_kv_heads=4, page_size=64, seed=92)
    d = ops.case_to_device(case, "cuda")
    kw = dict(sliding_window=64, mask_value=-30.0)
    _assert_close(_run(d, case, **kw), _ref(case, **kw), "window + mask -30")


# ------------------------------------------------------------------------------------- soft cap
@pytest.mark.parametrize("page,q_lens,kv_lens", [(64, [1, 1, 1], [700, 64, 3000]), (16, [1, 3, 1], [77, 300, 9]),
                                                 (64, [256, 1], [900, 400])])
def test_negative_soft_cap(cuda, page, q_lens, kv_lens):
    """soft_cap * tanh(s / soft_cap) for a negative cap equals |cap| * tanh(s / |cap|) (the reference
    rejects only 0.0); on the full-line decode path, the per-key path and a prefill-tile batch."""
    _say(f"soft_cap=-5 page={page} q_lens={q_lens}")
    case = make_custom(kv_lens=kv_lens, q_lens=q_lens, num_q_heads=32, num_kv_heads=8, page_size=page,
                       seed=page + sum(q_lens))
    d = ops.case_to_device(case, "cuda")
    got = _run(d, case, soft_cap=-5.0)
    _assert_close(got, _ref(case, soft_cap=-5.0), "soft_cap=-5")
    assert np.array_equal(got, _run(d, case, soft_cap=5.0))


# ------------------------------------------------------------------------------------- bad pages
@pytest.mark.parametrize("page", [64, 16])
def test_out_of_range_page_id_reads_page_zero_and_sets_the_error_word(cuda, page):
    """Documented behaviour of rpa.h: an out-of-range page id is never dereferenced; its rows are
    computed from page 0 instead, and bit 0 of the error word is set.  Other sequences are exact."""
    _say(f"out-of-range page id, page={page}")
    case = make_custom(kv_lens=[300, 500, 90], q_lens=[1, 1, 1], num_q_heads=16, num_kv_heads=4, page_size=page,
                       seed=95 + page)
    bad = case.page_indices.copy()
    bad[1, 2] = case.kv_pages.shape[0] + 7
    d = ops.case_to_device(case, "cuda")
    d["page_indices"] = torch.from_numpy(bad).cuda()
    torch.cuda.synchronize()
    with torch.cuda.stream(torch.cuda.Stream()):  # a fresh workspace: its error word starts at 0
        got = _run(d, case)
        assert ops.read_error_word() == 1
        d["page_indices"] = torch.from_numpy(case.page_indices).cuda()
        ok = _run(d, case)
    _assert_close(ok, _ref(case), "valid page ids")
    as_zero = bad.copy()
    as_zero[1, 2] = 0
    ref = orc.bf16_round(orc.ref_ragged_paged_attention(case.q, case.kv_pages, case.kv_lens, as_zero,
                                                        case.cu_q_lens, case.num_seqs, sm_scale=case.sm_scale))
    _assert_close(got, ref, "rows computed from page 0")


# ------------------------------------------------------------------------------------- GQA shapes
@pytest.mark.parametrize("hq,hkv", [(28, 4), (40, 8), (21, 3), (30, 5), (36, 6), (42, 7), (36, 12)])
def test_non_power_of_two_groups(cuda, hq, hkv):
    """G = 7, 5, 3, 6 and kv-head groups of 3, 5, 6, 7 waves: decode rows and a 300-token chunk."""
    _say(f"hq={hq} hkv={hkv}: decode + 300-token prefill")
    case = make_custom(kv_lens=[1000, 300, 45, 2500], q_lens=[1, 300, 1, 17], num_q_heads=hq, num_kv_heads=hkv,
                       page_size=64, seed=hq * 10 + hkv)
    d = ops.case_to_device(case, "cuda")
    _assert_close(_run(d, case), _ref(case), f"G={hq // hkv}")


# ------------------------------------------------------------------------------------- long
def test_c5_longest_sequence_131072_keys(cuda):
    """One sequence at C5's clip (131072 keys, PPS 2048) among short ones, C5's heads and page size."""
    _say("c5 shape with one 131072-key sequence")
    lens = [131072, 16, 900, 40, 5000, 17, 300, 2]
    case = make_custom(kv_lens=lens, q_lens=[1] * len(lens), num_q_heads=64, num_kv_heads=8, page_size=64,
                       pages_per_seq=2048, seed=131)
    d = ops.case_to_device(case, "cuda")
    _assert_close(_run(d, case), _ref(case), "131072 keys")


# ------------------------------------------------------------------------------------- prefill kernel
@pytest.mark.parametrize("hq,hkv,q_lens,kv_lens,page", [
    (32, 8, [512, 1, 300, 1], [1536, 900, 300, 77], 64),   # G=4: 64-token tiles, prior 1024 / none
    (64, 8, [100, 1, 17], [100, 4000, 50], 128),           # G=8: 32-token tiles, q_len == kv_len, page 128
    (8, 8, [300, 2], [337, 2], 64),                        # G=1: 256-token tiles
    (128, 8, [40, 1], [1040, 8], 64),                      # G=16: 16-token tiles
    (40, 8, [300, 1, 16], [3000, 600, 16], 64),            # G=5: 51-token tiles, one row per tile unused
    (12, 4, [700, 64], [2000, 64], 64),                    # 4 kv heads (no 8-wave workgroup needed)
    (32, 8, [2048], [6000], 64),                           # one long chunk: tiles split over many workgroups
])
def test_prefill_kernel_matches_oracle_and_other_paths(cuda, hq, hkv, q_lens, kv_lens, page):
    _say(f"prefill kernel hq={hq} hkv={hkv} q={q_lens} kv={kv_lens} page={page}")
    case = make_custom(kv_lens=kv_lens, q_lens=q_lens, num_q_heads=hq, num_kv_heads=hkv, page_size=page,
                       seed=sum(q_lens) + hq + page)
    d = ops.case_to_device(case, "cuda")
    ref = _ref(case)
    got = _run(d, case, prefill_tiles=1)
    _assert_close(got, ref, "prefill kernel")
    _assert_close(got, _run(d, case, prefill_tiles=-1)[: ref.shape[0]], "vs stream-K rows")
    assert np.array_equal(got, _run(d, case, prefill_tiles=1)), "not deterministic"


@pytest.mark.parametrize("kw", [dict(sliding_window=100), dict(soft_cap=30.0), dict(sliding_window=700, soft_cap=-8.0)])
def test_prefill_kernel_window_and_soft_cap(cuda, kw):
    _say(f"prefill kernel {kw}")
    case = make_custom(kv_lens=[2500, 300, 900], q_lens=[400, 1, 300], num_q_heads=32, num_kv_heads=8,
                       page_size=64, seed=77)
    d = ops.case_to_device(case, "cuda")
    _assert_close(_run(d, case, prefill_tiles=1, **kw), _ref(case, **kw), f"prefill kernel {kw}")


@pytest.mark.parametrize("wpc", [0, 2, 5])
def test_prefill_kernel_on_c3_with_other_knobs(cuda, c3_case, wpc):
    case, d, ref = c3_case
    _say(f"c3 prefill kernel, waves_per_cu={wpc}; in-kernel tiles")
    a = _run(d, case, prefill_tiles=1, waves_per_cu=wpc)
    _assert_close(a, ref, "prefill kernel")
    _assert_close(_run(d, case, prefill_tiles=2, waves_per_cu=wpc), ref, "in-kernel tiles")


def test_prefill_kernel_back_to_back_calls_leave_no_state(cuda):
    """Consecutive calls with different tile splits: every split descriptor is cleared by the merge."""
    _say("prefill kernel back-to-back")
    for i, (q, kv) in enumerate([([512, 512], [4000, 600]), ([64, 1, 1000], [64, 5000, 3000]), ([512, 512], [4000, 600])]):
        case = make_custom(kv_lens=kv, q_lens=q, num_q_heads=32, num_kv_heads=8, page_size=64, seed=400 + i)
        d = ops.case_to_device(case, "cuda")
        _assert_close(_run(d, case, prefill_tiles=1), _ref(case), f"call {i}")
    assert ops.read_error_word() == 0


def test_metadata_on_the_host_is_rejected_after_a_cached_call(cuda):
    """The wrapper caches its checks per call signature; the signature includes every tensor's
    device, so metadata moved to the host after a valid call is refused before any launch."""
    _say("host metadata after a cached call")
    case = make_custom(kv_lens=[100, 30], q_lens=[1, 1], num_q_heads=8, num_kv_heads=2, page_size=16, seed=501)
    d = ops.case_to_device(case, "cuda")
    _run(d, case)
    bad = dict(d, kv_lens=d["kv_lens"].cpu())
    with pytest.raises(ValueError, match="kv_lens must be on a GPU"):
        _run(bad, case)
    _assert_close(_run(d, case), _ref(case), "after the refusal")


# ------------------------------------------------------------------------------------- layouts
def test_split_co_tiles_then_prefill_kernel_then_co(cuda):
    """The co-resident layout splitting long tiles (a 17-token chunk over 4000 prior keys, priors
    that make 30-chunk tiles), then the prefill kernel on the same workspace, then the co layout
    again: each layout's merge descriptors stay apart (fields one leaves behind never read as the
    other's flags), every call within 2e-2 of the oracle."""
    case = make_custom(kv_lens=[1000, 1300, 45, 4017, 2200], q_lens=[1, 300, 1, 17, 64], num_q_heads=32,
                       num_kv_heads=8, page_size=64, seed=808)
    d = ops.case_to_device(case, "cuda")
    ref = _ref(case)
    _say("co-resident layout, split tiles")
    _assert_close(_run(d, case), ref, "co")
    _say("prefill kernel on the same workspace")
    _assert_close(_run(d, case, prefill_tiles=1), ref, "prefill kernel")
    _say("one 8-wave workgroup per CU")
    _assert_close(_run(d, case, prefill_tiles=3), ref, "8-wave tiles")
    _say("co-resident layout again")
    _assert_close(_run(d, case), ref, "co again")
    g3 = make_custom(kv_lens=[1000, 300, 45, 2500], q_lens=[1, 300, 1, 17], num_q_heads=21, num_kv_heads=3,
                     page_size=64, seed=213)
    _say("G=7 (prefill kernel) after the co layout's splits")
    _assert_close(_run(ops.case_to_device(g3, "cuda"), g3), _ref(g3), "G=7 after co")

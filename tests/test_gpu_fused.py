"""GPU parity of the fused Inkling decode (rpa_inkling_fused_decode through tpu_cake_amd.fused)
against the fused oracle, with the reference's gate (rpa_runner.py:112-122): output allclose at
0.02/0.02 and the updated cache bit-exact."""

import math
import sys

import numpy as np
import pytest
import torch

from oracle import rpa_fused_oracle as fo
from oracle import rpa_oracle as orc
from tpu_cake_amd import fused

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _to_device(inp):
    out = []
    for name in fused.INPUT_NAMES:
        a = inp[name]
        if a.dtype == np.uint16:
            t = torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
        else:
            t = torch.from_numpy(np.ascontiguousarray(a))
        out.append(t.cuda())
    return out


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def _run_and_check(inp):
    expected = fo.inkling_fused_rpa_reference(inp)
    args = _to_device(inp)
    out, cache = fused.run_preflighted(*args)
    torch.cuda.synchronize()
    got = (_bits(out), _bits(cache).reshape(inp["cache"].shape))
    err = orc.errors(orc.bf16_to_f32(got[0]), orc.bf16_to_f32(expected[0]))
    same_cache = np.array_equal(got[1], expected[1])
    print(f"  max_abs={err['max_abs']:.3e} cache_exact={same_cache}")
    assert same_cache
    assert fo.fused_rpa_outputs_pass(got, expected)
    assert fused.read_error_word() == 0
    return got


@pytest.mark.parametrize("seed", [97, 83, 0])
def test_reference_fixture(cuda, seed):
    _say(f"fused fixture seed {seed}")
    _run_and_check(fo.inkling_fused_rpa_inputs(seed=seed))


@pytest.mark.parametrize("hq,hkv,d,page,lens", [
    (32, 8, 128, 64, [1, 63, 64, 65, 511, 512, 513, 700, 2048, 3000]),   # Inkling decode shapes, D = 128
    (16, 4, 64, 16, [5, 16, 17, 300, 1000]),                             # narrower rows (D < 128)
    (8, 8, 128, 32, [2, 33, 100]),                                       # G = 1
])
def test_decode_shapes(cuda, hq, hkv, d, page, lens):
    _say(f"fused decode hq={hq} hkv={hkv} d={d} page={page}")
    pool = int(sum(-(-x // page) for x in lens) * 1.25) + 2
    inp = fo.fused_inputs_like(len(lens) * 7 + hq, nseq=len(lens), hq=hq, hkv=hkv, d=d, page_size=page,
                               pool_pages=pool, lengths=lens, rel_dim=16, extent=512)
    _run_and_check(inp)


@pytest.mark.parametrize("hq,hkv,page,lens,rel_dim,extent", [
    # one attention launch: no relative bias; windows of 40 and 8 distances (groups of 8)
    (32, 8, 64, [1, 31, 32, 33, 96, 700], 0, 512),
    (32, 8, 64, [1, 9, 40, 41, 300, 1025], 16, 40),
    (16, 2, 128, [2, 8, 129, 257], 16, 8),
    (64, 16, 64, [3, 64, 128, 130, 900], 16, 512),   # two kv-head groups (Hkv 16): heads 8..15 in the second
    (32, 8, 32, [32, 33, 64, 97], 16, 16),            # page 32: every unit its own page; window of 16
    # the prep launch: a window that is not a multiple of 8, a 32-wide projection
    (32, 8, 64, [5, 70, 200], 16, 20),
    (32, 8, 64, [5, 70, 200], 32, 64),
    (32, 8, 64, [5, 70, 200], 64, 64),                # R = 64 (the reference's fused core takes 16 only)
])
def test_bias_windows_and_launch_forms(cuda, hq, hkv, page, lens, rel_dim, extent):
    """Relative-bias windows at chunk edges and both forms of the call: the one-launch path (R in
    {0, 16}, E a multiple of 8) and the prep launch."""
    _say(f"fused bias hq={hq} hkv={hkv} page={page} R={rel_dim} E={extent}")
    pool = int(sum(-(-x // page) for x in lens) * 1.25) + 2
    inp = fo.fused_inputs_like(rel_dim * 5 + extent + page, nseq=len(lens), hq=hq, hkv=hkv, d=128,
                               page_size=page, pool_pages=pool, lengths=lens, rel_dim=rel_dim, extent=extent)
    _run_and_check(inp)


@pytest.mark.parametrize("hq,hkv,d,page,lens,rel_dim", [
    # one attention launch at head dims below 128 (queries, new rows and output that wide; the
    # cache rows 128, zero past d)
    (32, 8, 64, 64, [1, 31, 32, 33, 96, 700, 2048], 16),
    (16, 4, 96, 32, [2, 33, 64, 65, 1000], 0),
    (16, 4, 32, 64, [5, 64, 65, 300, 1500], 16),
    (8, 2, 120, 128, [3, 129, 257, 900], 16),
])
def test_one_launch_narrow_head_dims(cuda, hq, hkv, d, page, lens, rel_dim):
    _say(f"fused one launch d={d} hq={hq} hkv={hkv} page={page} R={rel_dim}")
    pool = int(sum(-(-x // page) for x in lens) * 1.25) + 2
    inp = fo.fused_inputs_like(d * 3 + page + rel_dim, nseq=len(lens), hq=hq, hkv=hkv, d=d, page_size=page,
                               pool_pages=pool, lengths=lens, rel_dim=rel_dim, extent=512)
    _run_and_check(inp)


def test_random_one_launch_sweep(cuda):
    """Seeded random shapes of the one-launch form (page 32/64/128, GQA 1-8, Hkv 1-16, R 0 or 16,
    E a multiple of 8 from 8 to 600, lengths 1-3000 incl. page and chunk edges) against the oracle
    at the reference's gate, cache bit-exact."""
    rng = np.random.default_rng(2024)
    for case in range(12):
        hkv = int(rng.choice([1, 2, 4, 8, 16]))
        g = int(rng.choice([1, 2, 4, 8]))
        page = int(rng.choice([32, 64, 128]))
        nseq = int(rng.integers(1, 24))
        lens = [int(x) for x in rng.integers(1, 3000, size=nseq)]
        lens[0] = int(rng.choice([1, 32, 33, page, page + 1]))
        rel = int(rng.choice([0, 16]))
        extent = 8 * int(rng.integers(1, 76))
        _say(f"fused sweep {case}: hq={hkv * g} hkv={hkv} page={page} nseq={nseq} R={rel} E={extent}")
        pool = int(sum(-(-x // page) for x in lens) * 1.25) + 2
        inp = fo.fused_inputs_like(100 + case, nseq=nseq, hq=hkv * g, hkv=hkv, d=128, page_size=page,
                                   pool_pages=pool, lengths=lens, rel_dim=rel, extent=extent)
        _run_and_check(inp)


@pytest.mark.parametrize("hq,hkv,d,page,lens,rel_dim,extent", [
    # one attention launch with pages smaller than a 32-key unit (each key's own page id): page 1 as
    # in the reference's sharded fixture, page 16 at unit and page edges, pages that do not divide 32
    (32, 8, 128, 1, [1, 2, 31, 32, 33, 300, 1000], 16, 512),
    (32, 8, 128, 16, [1, 15, 16, 17, 31, 32, 33, 64, 700, 2048], 16, 512),
    (16, 4, 64, 16, [5, 16, 17, 300, 1000], 0, 512),
    (32, 8, 128, 24, [1, 23, 24, 25, 48, 49, 500], 16, 40),
    (8, 8, 128, 8, [2, 9, 33, 100], 16, 8),
    (16, 2, 96, 48, [3, 47, 48, 49, 97, 1500], 16, 512),
])
def test_one_launch_small_pages(cuda, hq, hkv, d, page, lens, rel_dim, extent):
    _say(f"fused one launch page={page} d={d} hq={hq} hkv={hkv} R={rel_dim} E={extent}")
    pool = int(sum(-(-x // page) for x in lens) * 1.25) + 2
    inp = fo.fused_inputs_like(page * 7 + d + rel_dim, nseq=len(lens), hq=hq, hkv=hkv, d=d, page_size=page,
                               pool_pages=pool, lengths=lens, rel_dim=rel_dim, extent=extent)
    _run_and_check(inp)


def test_random_small_page_sweep(cuda):
    """Seeded random shapes of the one-launch form with pages of 1 to 31 keys (each key of a unit
    read from its own page), GQA 1-8, Hkv 1-16, R 0 or 16, head dims 32-128, cache bit-exact."""
    rng = np.random.default_rng(4048)
    for case in range(10):
        hkv = int(rng.choice([1, 2, 4, 8, 16]))
        g = int(rng.choice([1, 2, 4, 8]))
        page = int(rng.choice([1, 2, 4, 8, 12, 16, 20, 31]))
        d = int(rng.choice([32, 64, 128]))
        nseq = int(rng.integers(1, 20))
        lens = [int(x) for x in rng.integers(1, 1500, size=nseq)]
        lens[0] = int(rng.choice([1, 32, 33, page, page + 1]))
        rel = int(rng.choice([0, 16]))
        extent = 8 * int(rng.integers(1, 76))
        _say(f"fused small-page sweep {case}: hq={hkv * g} hkv={hkv} d={d} page={page} nseq={nseq} R={rel} E={extent}")
        pool = int(sum(-(-x // page) for x in lens) * 1.25) + 2
        inp = fo.fused_inputs_like(300 + case, nseq=nseq, hq=hkv * g, hkv=hkv, d=d, page_size=page,
                                   pool_pages=pool, lengths=lens, rel_dim=rel, extent=extent)
        _run_and_check(inp)


def test_more_than_256_sequences(cuda):
    """Metadata past the first four 64-sequence windows (loaded one window at a time)."""
    rng = np.random.default_rng(11)
    lens = [int(x) for x in rng.integers(1, 200, size=300)]
    _say("fused 300 sequences")
    pool = int(sum(-(-x // 32) for x in lens) * 1.25) + 2
    inp = fo.fused_inputs_like(12, nseq=300, hq=8, hkv=8, d=128, page_size=32, pool_pages=pool, lengths=lens,
                               rel_dim=16, extent=64)
    _run_and_check(inp)


def test_rejected_metadata_never_reaches_the_kernel(cuda):
    _say("fused preflight before the kernel")
    inp = fo.inkling_fused_rpa_inputs(seed=97)
    pages = inp["page_indices"].copy()
    pages[2] = pages[0]
    inp["page_indices"] = pages
    args = _to_device(inp)
    before = _bits(args[3]).copy()
    with pytest.raises(ValueError, match="updates collide"):
        fused.run_preflighted(*args)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(args[3]), before)


@pytest.mark.parametrize("bad,page", [(-64, 64), (5, 64), (-16, 16), (5, 16)])
def test_one_launch_drops_a_sequence_with_bad_page_offset(cuda, bad, page):
    """Metadata the preflight would reject, sent straight to the kernel (fused.invoke): a negative or
    unaligned cu_kv_lens entry drops that sequence (page bit of the error word, its cache slot left
    as it was) and leaves every other sequence's output and cache update as the oracle's."""
    _say(f"fused one launch, page {page}, cu_kv[1] = {bad}")
    lens = [40, 100, 70, 300]
    pool = int(sum(-(-x // page) for x in lens) * 1.25) + 2
    inp = fo.fused_inputs_like(5, nseq=4, hq=32, hkv=8, d=128, page_size=page, pool_pages=pool, lengths=lens,
                               rel_dim=16, extent=512)
    expected = fo.inkling_fused_rpa_reference(inp)
    bad_inp = dict(inp)
    cu = inp["cu_kv_lens"].copy()
    cu[1] = bad
    bad_inp["cu_kv_lens"] = cu
    args = _to_device(bad_inp)
    before = _bits(args[3]).copy().reshape(inp["cache"].shape)
    torch.cuda.synchronize()
    with torch.cuda.stream(torch.cuda.Stream()):  # a fresh workspace: its error word starts at 0
        out, cache = fused.invoke(*args)
        torch.cuda.current_stream().synchronize()
        assert fused.read_error_word() == 1
    torch.cuda.synchronize()
    got_o = orc.bf16_to_f32(_bits(out))
    exp_o = orc.bf16_to_f32(expected[0])
    keep = [0, 2, 3]
    assert np.allclose(got_o[keep], exp_o[keep], atol=0.02, rtol=0.02)
    got_c = _bits(cache).reshape(inp["cache"].shape)
    # sequence 1's slot: untouched; everything else: the oracle's updated cache
    pg = int(inp["page_indices"][int(inp["cu_kv_lens"][1]) // page + (lens[1] - 1) // page])
    slot = (lens[1] - 1) % page
    want = expected[1].copy()
    want[pg, slot] = before[pg, slot]
    assert np.array_equal(got_c, want)


def test_repeat_is_idempotent(cuda):
    """Writing the same token twice leaves the same cache and output."""
    _say("fused repeat")
    inp = fo.inkling_fused_rpa_inputs(seed=3)
    args = _to_device(inp)
    out1, cache1 = fused.run_preflighted(*args)
    o1, c1 = _bits(out1).copy(), _bits(cache1).copy()
    out2, cache2 = fused.run_preflighted(*args)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out2), o1) and np.array_equal(_bits(cache2), c1)

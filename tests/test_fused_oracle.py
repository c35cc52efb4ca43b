"""CPU pins for the fused Inkling decode oracle (oracle/rpa_fused_oracle.py).

The first two tests restate the reference's own tests (tests/test_rpa_oracle.py:10-39) and its
preflight cases (tests/test_rpa_lowering.py:604-653); the rest pin the oracle independently.
"""

import numpy as np
import pytest

from oracle import rpa_oracle as orc
from oracle import rpa_fused_oracle as fo


def test_seed_replay_shapes_and_cache_update():
    a = fo.inkling_fused_rpa_inputs(seed=83)
    b = fo.inkling_fused_rpa_inputs(seed=83)
    for k in a:
        assert np.array_equal(a[k], b[k]), k
    assert not np.array_equal(a["page_indices"], np.arange(32, dtype=np.int32))
    assert tuple(a["page_indices"][:6]) == (7, 2, 19, 4, 25, 1)
    out, cache = fo.inkling_fused_rpa_reference(a)
    assert out.shape == (4, 4, 32) and out.dtype == np.uint16
    assert cache.shape == (32, 16, 2, 2, 128) and cache.dtype == np.uint16
    assert not np.array_equal(cache, a["cache"])


def test_every_mutation_fails_the_gate():
    inp = fo.inkling_fused_rpa_inputs(seed=97)
    expected = fo.inkling_fused_rpa_reference(inp)
    assert fo.fused_rpa_outputs_pass(expected, expected)
    for m in fo.FUSED_MUTATIONS:
        wrong = fo.inkling_fused_rpa_reference(inp, mutation=m)
        assert not fo.fused_rpa_outputs_pass(wrong, expected), m


def test_gate_needs_exact_cache():
    # rpa_runner tests/test_rpa_runner.py:25-42: output within tolerance passes, any cache bit fails
    inp = fo.inkling_fused_rpa_inputs(seed=5)
    out, cache = fo.inkling_fused_rpa_reference(inp)
    bumped = orc.bf16_from_f32(orc.bf16_to_f32(out) + np.float32(0.001))
    assert fo.fused_rpa_outputs_pass((bumped, cache), (out, cache))
    c2 = cache.copy()
    c2.flat[12345] ^= 1
    assert not fo.fused_rpa_outputs_pass((out, c2), (out, cache))


def test_cache_changes_exactly_at_the_written_rows():
    inp = fo.inkling_fused_rpa_inputs(seed=11)
    _, cache = fo.inkling_fused_rpa_reference(inp)
    before = inp["cache"].reshape(32, 16, 4, 128)
    after = cache.reshape(32, 16, 4, 128)
    expect = before.copy()
    S = 16
    for s, length in enumerate(inp["kv_lengths"]):
        pos = int(length) - 1
        page = inp["page_indices"][inp["cu_kv_lens"][s] // S + pos // S]
        for h in range(2):
            for row, src in ((2 * h, inp["keys"]), (2 * h + 1, inp["values"])):
                expect[page, pos % S, row] = 0
                expect[page, pos % S, row, :32] = src[s, h]
    assert np.array_equal(after, expect)


def _as_rpa(inp, cache_bits):
    """The fused contract as an upstream RPA call: flat page list -> [N, PPS] table, the cache
    narrowed to the query width."""
    S = cache_bits.shape[1]
    nseq = len(inp["kv_lengths"])
    pps = int(max(-(-int(x) // S) for x in inp["kv_lengths"]))
    table = np.zeros((nseq, pps), np.int32)
    for s, length in enumerate(inp["kv_lengths"]):
        n = -(-int(length) // S)
        first = int(inp["cu_kv_lens"][s]) // S
        table[s, :n] = inp["page_indices"][first:first + n]
    d = inp["queries"].shape[-1]
    kv = cache_bits.reshape(cache_bits.shape[0], S, -1, cache_bits.shape[-1])[..., :d]
    return kv, table


def test_zero_relative_states_equal_the_rpa_oracle():
    inp = fo.inkling_fused_rpa_inputs(seed=23)
    inp["relative_states"] = np.zeros_like(inp["relative_states"])
    out, cache = fo.inkling_fused_rpa_reference(inp)
    kv, table = _as_rpa(inp, cache)
    ref = orc.ref_ragged_paged_attention(inp["queries"], kv, inp["kv_lengths"], table, inp["cu_q_lens"],
                                         np.array([4], np.int32), sm_scale=1.0 / 32, probs_bf16=False)
    err = orc.errors(orc.bf16_to_f32(out), orc.bf16_round(ref))
    assert err["max_abs"] <= 8e-3, err


def test_single_key_returns_the_new_value_row():
    inp = fo.inkling_fused_rpa_inputs(seed=29)  # sequence 0 has kv_len 1: its only key is the new token
    out, _ = fo.inkling_fused_rpa_reference(inp)
    for h in range(4):
        assert np.array_equal(out[0, h], inp["values"][0, h // 2])


@pytest.mark.parametrize("distance", [0, 5, 16])
def test_bias_selects_the_key_at_its_distance(distance):
    """A projection that is 60 at one distance and 0 elsewhere, unit relative states: the output
    is (almost exactly) the V row of the key that far from the newest one."""
    inp = fo.inkling_fused_rpa_inputs(seed=31)
    proj = np.zeros((16, 128), np.float32)
    proj[0, distance] = 60.0
    inp["relative_projection"] = orc.bf16_from_f32(proj)
    rs = np.zeros((4, 4, 16), np.float32)
    rs[:, :, 0] = 1.0
    inp["relative_states"] = orc.bf16_from_f32(rs)
    inp["queries"] = orc.bf16_from_f32(np.zeros((4, 4, 32), np.float32))
    out, cache = fo.inkling_fused_rpa_reference(inp)
    S = 16
    flat = orc.bf16_to_f32(cache).reshape(32, S, 4, 128)
    s = 3  # kv_len 49
    length = int(inp["kv_lengths"][s])
    key = length - 1 - distance
    page = inp["page_indices"][inp["cu_kv_lens"][s] // S + key // S]
    for h in range(4):
        v = flat[page, key % S, 2 * (h // 2) + 1, :32]
        assert np.allclose(orc.bf16_to_f32(out[s, h]), v, atol=1e-2)


def _preflight_cases():
    base = fo.inkling_fused_rpa_inputs(seed=0)
    cases = []
    c = dict(base, distribution=np.zeros((3,), np.int32))
    cases.append((c, "decode-only distribution"))
    c = dict(base, page_indices=np.full((32,), 99, np.int32))
    cases.append((c, "outside the fused cache"))
    pages = base["page_indices"].copy()
    pages[2] = pages[0]
    cases.append((dict(base, page_indices=pages), "updates collide"))
    pages = base["page_indices"].copy()
    pages[2] = pages[1]
    cases.append((dict(base, page_indices=pages), "aliases logical pages"))
    pages = base["page_indices"].copy()
    pages[1] = pages[0]
    cases.append((dict(base, kv_lengths=np.asarray((1, 2, 33, 49), np.int32), page_indices=pages,
                       cu_kv_lens=np.asarray((0, 16, 32, 80, 144), np.int32)), "active write page is shared"))
    big = np.iinfo(np.int32)
    cases.append((dict(base, kv_lengths=np.full((4,), big.max, np.int32),
                       cu_kv_lens=np.asarray((0, big.min, 0, big.min, 0), np.int32)), "exceeds total cache capacity"))
    cases.append((dict(base, cu_q_lens=np.asarray((0, 1, 2, 3, 5), np.int32)), "one query token per sequence"))
    cases.append((dict(base, kv_lengths=np.asarray((0, 17, 33, 49), np.int32)), "positive KV lengths"))
    cases.append((dict(base, cu_kv_lens=np.asarray((0, 17, 48, 96, 160), np.int32)), "page-aligned"))
    return base, cases


def test_preflight_accepts_the_fixture_and_rejects_bad_metadata():
    base, cases = _preflight_cases()
    fo.preflight_fused_decode(base)
    for inp, msg in cases:
        with pytest.raises(ValueError, match=msg):
            fo.preflight_fused_decode(inp)


def test_larger_fixture_passes_preflight():
    inp = fo.fused_inputs_like(3, nseq=6, hq=32, hkv=8, d=128, page_size=64, pool_pages=40,
                               lengths=[1, 63, 64, 65, 700, 1000], rel_dim=16, extent=512)
    fo.preflight_fused_decode(inp)
    out, cache = fo.inkling_fused_rpa_reference(inp)
    assert out.shape == (6, 32, 128) and np.isfinite(orc.bf16_to_f32(out)).all()
    assert np.count_nonzero(cache != inp["cache"]) > 0

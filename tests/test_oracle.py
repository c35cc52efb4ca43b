"""Pins the CPU oracle (oracle/rpa_oracle.py) against the reference's known answers,
closed forms, brute force and a mutation catalogue -- each chosen so that a plausible
mistake (dropped term, wrong index, swapped operand) fails one of them."""

import math

import numpy as np
import pytest
import torch

from oracle import rpa_oracle as orc

TOL = 2e-2


# ---------------------------------------------------------------- number formats
def test_bf16_decode_encode_exhaustive():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = orc.bf16_to_f32(bits)
    t = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    finite = np.isfinite(t)
    assert np.array_equal(f[finite], t[finite])
    assert np.array_equal(np.isnan(f), np.isnan(t))
    back = orc.bf16_from_f32(f)
    assert np.array_equal(back[finite], bits[finite])


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(500_000).astype(np.float32),
        (rng.standard_normal(200_000) * 1e30).astype(np.float32),
        (rng.standard_normal(200_000) * 1e-30).astype(np.float32),
        # exact ties: low 16 bits 0x8000
        (rng.integers(0, 1 << 15, 100_000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ])
    x = x[np.isfinite(x)]
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.bf16_from_f32(x), want)


def test_fp8_decode_closed_form_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    v = orc.fp8e4m3_to_f32(codes)
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            assert np.isnan(v[c])
            continue
        mag = (m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
        assert v[c] == (-mag if s else mag), c
    assert orc.fp8e4m3_to_f32(np.array([0x7E], np.uint8))[0] == 448.0


def test_fp8_encode_roundtrip_and_nearest_even():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    assert np.array_equal(orc.fp8e4m3_from_f32(orc.fp8e4m3_to_f32(codes)), codes)
    # saturation and ties
    assert orc.fp8e4m3_from_f32(np.array([1000.0, -1e9], np.float32)).tolist() == [0x7E, 0xFE]
    one, nxt = 1.0, 1.125  # adjacent codes 0x38 (even mantissa) and 0x39
    assert orc.fp8e4m3_from_f32(np.array([(one + nxt) / 2], np.float32))[0] == 0x38
    # agrees with torch's e4m3fn cast in range
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(200_000) * 60).astype(np.float32)
    x = np.clip(x, -448, 448)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(orc.fp8e4m3_from_f32(x), want)


# ---------------------------------------------------------------- helpers
def _case(lens, qlens, hq, hkv, d=128, page=16, seed=0, scale=None, pool_factor=1.5):
    rng = np.random.default_rng(seed)
    need = sum(-(-l // page) for l in lens)
    P = max(1, int(math.ceil(pool_factor * need)))
    pps = max(1, max(-(-l // page) for l in lens))
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((len(lens), pps), np.int32)
    off = 0
    for i, l in enumerate(lens):
        n = -(-l // page)
        table[i, :n] = perm[off: off + n]
        off += n
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    q = orc.bf16_from_f32(rng.standard_normal((cu[-1], hq, d)).astype(np.float32))
    kv = orc.bf16_from_f32(rng.standard_normal((P, page, 2 * hkv, d)).astype(np.float32))
    return dict(q_bits=q, kv_pages=kv, kv_lens=np.array(lens, np.int32), page_indices=table, cu_q_lens=cu,
                num_seqs=np.array([len(lens)], np.int32)), (scale if scale is not None else 1 / math.sqrt(d))


def _dense(case, i):
    k, v, _ = orc.gather_kv(case["kv_pages"], case["page_indices"], int(case["kv_lens"][i]), i)
    return orc.bf16_to_f32(k), orc.bf16_to_f32(v)


# ---------------------------------------------------------------- known answers
def test_reference_known_answer_inkling():
    """tests/test_workloads.py:42-60 of the reference, through the restated numpy oracle."""
    query = np.ones((1, 4, 8), dtype=np.float32)
    key_cache = np.ones((2, 4, 2, 8), dtype=np.float32)
    value_cache = np.arange(2 * 4 * 1 * 6, dtype=np.float32).reshape(2, 4, 1, 6)
    out = orc.inkling_rpa_reference(query, key_cache, value_cache, np.array([[0, 1]], np.int32),
                                    np.array([5], np.int32), np.zeros((4, 8), np.float32))
    assert out.shape == (1, 4, 6)
    np.testing.assert_allclose(out[0], np.broadcast_to(np.arange(6) + 12, (4, 6)))


def _inkling_case(seed, hq=8, hk=2, d=32, lens=(1, 17, 40), page=8, pool=24):
    """bf16-representable inputs for the Inkling oracle and the same data in the operator layout
    (K of kv head h at combined head 2h, V at 2h+1; one query token per sequence)."""
    g = np.random.default_rng(seed)
    rnd = lambda *shape: orc.bf16_round(g.normal(size=shape).astype(np.float32))
    query, kc, vc = rnd(len(lens), hq, d), rnd(pool, page, hk, d), rnd(pool, page, hk, d)
    mp = max(-(-L // page) for L in lens)
    perm = g.permutation(pool).astype(np.int32)
    table = np.zeros((len(lens), mp), np.int32)
    off = 0
    for i, L in enumerate(lens):
        n = -(-L // page)
        table[i, :n] = perm[off:off + n]
        off += n
    lengths = np.asarray(lens, np.int32)
    kv = np.empty((pool, page, 2 * hk, d), np.float32)
    kv[:, :, 0::2], kv[:, :, 1::2] = kc, vc
    op = dict(q_bits=orc.bf16_from_f32(query), kv_pages=orc.bf16_from_f32(kv), kv_lens=lengths,
              page_indices=table, cu_q_lens=np.arange(len(lens) + 1, dtype=np.int32),
              num_seqs=np.array([len(lens)], np.int32))
    return (query, kc, vc, table, lengths), op


def test_inkling_reference_zero_bias_is_rpa_at_scale_one_over_d():
    """With a zero bias the Inkling oracle (scale 1/D, inkling_rpa.py:68) is the upstream operator's
    oracle at sm_scale = 1/D with fp32 probabilities, over distinct K and V heads, shuffled pages
    and ragged lengths; at 1/sqrt(D) it is not (the slip this pins)."""
    (query, kc, vc, table, lengths), op = _inkling_case(3)
    d = query.shape[-1]
    zero = np.zeros((query.shape[1], int(lengths.max())), np.float32)
    got = orc.inkling_rpa_reference(query, kc, vc, table, lengths, zero)
    ref = orc.ref_ragged_paged_attention(**op, sm_scale=1.0 / d, probs_bf16=False)
    assert np.allclose(got, ref, atol=2e-5, rtol=2e-5)
    # and the brute-force dense attention, GQA-expanded, per sequence
    kmap = np.arange(query.shape[1]) // (query.shape[1] // kc.shape[2])
    for b, L in enumerate(lengths.tolist()):
        keys = kc[table[b, : -(-L // kc.shape[1])]].reshape(-1, kc.shape[2], d)[:L][:, kmap]
        vals = vc[table[b, : -(-L // vc.shape[1])]].reshape(-1, vc.shape[2], d)[:L][:, kmap]
        dense = orc.dense_attention_f64(query[b][None].astype(np.float64), keys.astype(np.float64),
                                        vals.astype(np.float64), 1.0 / d, None)[0]
        assert np.allclose(got[b], dense, atol=2e-5, rtol=2e-5)
    wrong = orc.ref_ragged_paged_attention(**op, sm_scale=1.0 / np.sqrt(d), probs_bf16=False)
    assert np.abs(got - wrong).max() > 0.05


def test_inkling_reference_bias_selects_and_adds_by_key_position():
    """A one-hot bias (+60 at key l_h of head h) makes head h return V row l_h of its kv head: the
    bias is indexed [head, key position] and added to the scaled scores.  A small random bias
    shifts the result exactly as adding it to the upstream oracle's scores would (mask_value
    path: bias b -> softmax over s/D + b)."""
    (query, kc, vc, table, lengths), op = _inkling_case(5)
    hq, d = query.shape[1], query.shape[2]
    hk = kc.shape[2]
    L = int(lengths.max())
    bias = np.zeros((hq, L), np.float32)
    pick = [(7 * h + 3) % int(lengths.min()) for h in range(hq)]
    for h in range(hq):
        bias[h, pick[h]] = 60.0
    got = orc.inkling_rpa_reference(query, kc, vc, table, lengths, bias)
    for b, Lb in enumerate(lengths.tolist()):
        vals = vc[table[b, : -(-Lb // vc.shape[1])]].reshape(-1, hk, d)[:Lb]
        for h in range(hq):
            assert np.allclose(got[b, h], vals[pick[h], h // (hq // hk)], atol=1e-5)
    # transposing the bias (indexing it [key, head]) would pick other rows
    small = np.random.default_rng(9).normal(scale=0.3, size=(hq, L)).astype(np.float32)
    got = orc.inkling_rpa_reference(query, kc, vc, table, lengths, small)
    kmap = np.arange(hq) // (hq // hk)
    for b, Lb in enumerate(lengths.tolist()):
        keys = kc[table[b, : -(-Lb // kc.shape[1])]].reshape(-1, hk, d)[:Lb][:, kmap].astype(np.float64)
        vals = vc[table[b, : -(-Lb // vc.shape[1])]].reshape(-1, hk, d)[:Lb][:, kmap].astype(np.float64)
        s = np.einsum("hd,lhd->hl", query[b].astype(np.float64), keys) / d + small[:, :Lb]
        w = np.exp(s - s.max(axis=1, keepdims=True))
        w /= w.sum(axis=1, keepdims=True)
        assert np.allclose(got[b], np.einsum("hl,lhd->hd", w, vals), atol=2e-5)


def test_inkling_reference_deterministic_and_finite():
    inputs = orc.inkling_rpa_inputs()
    a = orc.inkling_rpa_reference(*inputs)
    b = orc.inkling_rpa_reference(*inputs)
    assert np.array_equal(a, b) and a.shape == (4, 4, 32) and np.isfinite(a).all()


def test_uniform_keys_give_mean_of_values():
    case, sc = _case([37], [1], 8, 2)
    case["kv_pages"][:, :, 0::2, :] = orc.bf16_from_f32(np.ones(1, np.float32))[0]  # all K = 1
    out = orc.ref_ragged_paged_attention(**case, sm_scale=sc, probs_bf16=False)
    _, v = _dense(case, 0)
    want = v.mean(axis=0)[np.arange(8) // 4]
    np.testing.assert_allclose(out[0], want, atol=1e-5)


def test_single_key_returns_value_row():
    case, sc = _case([1, 1], [1, 1], 4, 4)
    out = orc.ref_ragged_paged_attention(**case, sm_scale=sc)
    for i in range(2):
        _, v = _dense(case, i)
        np.testing.assert_array_equal(out[i], v[0])


def test_one_hot_logit_selects_value():
    case, sc = _case([40], [1], 2, 1, seed=3)
    k = np.zeros((40, 128), np.float32)
    k[17] = 1.0
    q = np.full((1, 2, 128), 8.0, np.float32)
    case["q_bits"] = orc.bf16_from_f32(q)
    pages = case["page_indices"][0]
    for t in range(40):
        case["kv_pages"][pages[t // 16], t % 16, 0] = orc.bf16_from_f32(k[t])
    out = orc.ref_ragged_paged_attention(**case, sm_scale=1.0, probs_bf16=False)
    _, v = _dense(case, 0)
    np.testing.assert_allclose(out[0, 0], v[17, 0], atol=1e-6)


# ---------------------------------------------------------------- brute force / textbook
def test_matches_dense_brute_force_mixed_batch():
    lens, qlens = [9, 33, 20], [1, 5, 20]
    case, sc = _case(lens, qlens, 4, 2, d=32, seed=5)
    out = orc.ref_ragged_paged_attention(**case, sm_scale=sc, probs_bf16=False)
    q_all = orc.bf16_to_f32(case["q_bits"]).astype(np.float64)
    for i, (L, ql) in enumerate(zip(lens, qlens)):
        k, v = _dense(case, i)
        kk, vv = k[:, np.arange(4) // 2].astype(np.float64), v[:, np.arange(4) // 2].astype(np.float64)
        c0 = case["cu_q_lens"][i]
        want = orc.dense_attention_f64(q_all[c0:c0 + ql], kk, vv, sc, causal_offset=L - ql)
        np.testing.assert_allclose(out[c0:c0 + ql], want, atol=2e-6)


def test_causal_self_attention_when_q_len_equals_kv_len():
    case, sc = _case([12], [12], 2, 2, d=16, seed=6)
    out = orc.ref_ragged_paged_attention(**case, sm_scale=sc, probs_bf16=False)
    q = orc.bf16_to_f32(case["q_bits"]).astype(np.float64)
    k, v = _dense(case, 0)
    for j in range(12):  # row j sees keys 0..j only
        for h in range(2):
            s = (k[: j + 1, h] @ q[j, h]) * sc
            w = np.exp(s - s.max())
            w /= w.sum()
            np.testing.assert_allclose(out[j, h], w @ v[: j + 1, h], atol=2e-6)


def test_gqa_mapping_with_distinct_values_per_head():
    case, sc = _case([25], [1], 8, 4, seed=7)
    out = orc.ref_ragged_paged_attention(**case, sm_scale=sc, probs_bf16=False)
    q = orc.bf16_to_f32(case["q_bits"]).astype(np.float64)
    k, v = _dense(case, 0)
    for h in range(8):
        kvh = h // 2
        s = k[:, kvh] @ q[0, h] * sc
        w = np.exp(s - s.max())
        w /= w.sum()
        np.testing.assert_allclose(out[0, h], w @ v[:, kvh], atol=2e-6)


def test_sliding_window_and_soft_cap_closed_form():
    case, sc = _case([30], [3], 2, 2, d=16, seed=8)
    out = orc.ref_ragged_paged_attention(**case, sm_scale=sc, probs_bf16=False, sliding_window=5, soft_cap=2.0)
    q = orc.bf16_to_f32(case["q_bits"]).astype(np.float64)
    k, v = _dense(case, 0)
    for j in range(3):
        pos = 27 + j
        keys = np.arange(pos - 4, pos + 1)  # window 5: keys pos-4 .. pos
        for h in range(2):
            s = 2.0 * np.tanh((k[keys, h] @ q[j, h]) * sc / 2.0)
            w = np.exp(s - s.max())
            w /= w.sum()
            np.testing.assert_allclose(out[j, h], w @ v[keys, h], atol=2e-6)


# ---------------------------------------------------------------- gather / permutation
def test_gather_matches_independent_dense_layout():
    case, _ = _case([5, 40, 17], [1, 1, 1], 4, 2, page=8, seed=9)
    for i, L in enumerate([5, 40, 17]):
        k, v, pages = orc.gather_kv(case["kv_pages"], case["page_indices"], L, i)
        for t in range(L):
            p = case["page_indices"][i, t // 8]
            assert np.array_equal(k[t], case["kv_pages"][p, t % 8, 0::2])
            assert np.array_equal(v[t], case["kv_pages"][p, t % 8, 1::2])
        assert len(pages) == -(-L // 8)


def test_page_pool_permutation_invariance():
    case, sc = _case([50, 3, 77], [1, 2, 1], 4, 2, seed=10)
    a = orc.ref_ragged_paged_attention(**case, sm_scale=sc)
    P = case["kv_pages"].shape[0]
    sigma = np.random.default_rng(0).permutation(P)
    inv = np.argsort(sigma)
    c2 = dict(case)
    c2["kv_pages"] = case["kv_pages"][inv]
    c2["page_indices"] = sigma[case["page_indices"]].astype(np.int32)
    b = orc.ref_ragged_paged_attention(**c2, sm_scale=sc)
    assert np.array_equal(a, b)


def test_fp8_with_per_page_scales_equals_dequantised_bf16():
    case, sc = _case([64, 10], [1, 1], 4, 2, seed=11)
    src = orc.bf16_to_f32(case["kv_pages"])
    P, S, C, D = src.shape
    x = src.reshape(P, S, 2, 2, D)
    amax = np.abs(x).max(axis=(1, 4))
    scale = np.where(amax > 0, amax / 448.0, 1.0).astype(np.float32)
    codes = orc.fp8e4m3_from_f32(x / scale[:, None, :, :, None]).reshape(P, S, C, D)
    out = orc.ref_ragged_paged_attention(**{**case, "kv_pages": codes}, sm_scale=sc, kv_scales=scale, kv_dtype="fp8")
    deq = orc.bf16_round((orc.fp8e4m3_to_f32(codes).reshape(P, S, 2, 2, D) * scale[:, None, :, :, None]).astype(np.float32))
    ref = orc.ref_ragged_paged_attention(**{**case, "kv_pages": deq.reshape(P, S, C, D)}, sm_scale=sc, kv_dtype="f32")
    np.testing.assert_allclose(out, ref, atol=1e-6)


# ---------------------------------------------------------------- mutation catalogue
@pytest.mark.parametrize("mutation", ["wrong_scale", "ignore_page_indices", "wrong_page_index",
                                      "swap_kv_interleave", "wrong_gqa_map", "no_causal_mask"])
def test_mutations_fail_the_tolerance(mutation):
    """Modelled on FusedRpaOracleMutation (workloads/inkling_rpa.py:404-410): every planted
    mistake must break the 2e-2 bar, so passing it means something."""
    case, sc = _case([200, 64, 33], [1, 16, 1], 8, 2, seed=12, scale=0.25)
    good = orc.ref_ragged_paged_attention(**case, sm_scale=sc)
    bad = orc.ref_ragged_paged_attention(**case, sm_scale=sc, _mutation=mutation)
    assert orc.errors(bad, good)["max_abs"] > TOL


# ---------------------------------------------------------------- validation
def test_static_validation_errors():
    case, _ = _case([5], [1], 4, 2)
    with pytest.raises(ValueError, match="must be divisible"):
        orc.static_validate_inputs((1, 3, 128), case["kv_pages"].shape, case["kv_lens"], case["page_indices"],
                                   case["cu_q_lens"], case["num_seqs"])
    with pytest.raises(ValueError, match="sliding_window"):
        orc.static_validate_inputs((1, 4, 128), case["kv_pages"].shape, case["kv_lens"], case["page_indices"],
                                   case["cu_q_lens"], case["num_seqs"], sliding_window=0)
    with pytest.raises(ValueError, match="soft_cap"):
        orc.static_validate_inputs((1, 4, 128), case["kv_pages"].shape, case["kv_lens"], case["page_indices"],
                                   case["cu_q_lens"], case["num_seqs"], soft_cap=0.0)


def test_dynamic_validation_errors():
    lens = np.array([10, 4], np.int32)
    table = np.zeros((2, 1), np.int32)
    with pytest.raises(ValueError, match="pages_per_seq"):
        orc.dynamic_validate_inputs(4, 8, lens, table, np.array([0, 1, 2], np.int32), np.array([2], np.int32))
    with pytest.raises(ValueError, match="q_len"):
        orc.dynamic_validate_inputs(8, 16, lens, table, np.array([0, 1, 7], np.int32), np.array([2], np.int32))
    with pytest.raises(ValueError, match="num_seqs"):
        orc.dynamic_validate_inputs(8, 16, lens, table, np.array([0, 1, 2], np.int32), np.array([3], np.int32))


def test_golden_fixture_reproduces():
    import pathlib
    import sys
    sys.path.insert(0, str(pathlib.Path(__file__).resolve().parents[1] / "tpu-cake_amd"))
    from tpu_cake_amd.workloads import make_config
    gold = np.load(pathlib.Path(__file__).parent / "golden" / "c1_expected.npz")
    case = make_config("c1", values="host")
    out = orc.ref_ragged_paged_attention(case.q, case.kv_pages, case.kv_lens, case.page_indices, case.cu_q_lens,
                                         case.num_seqs, sm_scale=case.sm_scale)
    assert np.array_equal(orc.bf16_from_f32(out), gold["out_bf16"])

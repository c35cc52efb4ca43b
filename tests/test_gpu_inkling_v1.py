"""The v1 Inkling decode contract (``experiment inkling-rpa``) on the GPU, through the C ABI
(``rpa_inkling_decode`` via ``tpu_cake_amd.inkling``), against the oracle
``oracle/rpa_oracle.py::inkling_rpa_reference`` (inkling_rpa.py:37-73) on the same bf16 inputs."""

import numpy as np
import pytest
import torch

from oracle import rpa_oracle as orc
from tpu_cake_amd import inkling

pytestmark = pytest.mark.gpu
TOL = 2e-2


@pytest.fixture(scope="module")
def cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)


def _say(msg):
    print(f"[case] {msg}", flush=True)


def to_device_bf16(bits, dev):
    """uint16 bf16 bit patterns -> a bf16 tensor on the device."""
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).copy()).view(torch.bfloat16).to(dev)


def _run(dev, query, key_cache, value_cache, page_table, lengths, bias):
    """bf16-round the float inputs, run GPU and oracle on the same values; returns (gpu, oracle)."""
    q, k, v, b = (orc.bf16_from_f32(np.asarray(x, np.float32)) for x in (query, key_cache, value_cache, bias))
    args = [to_device_bf16(x, dev) for x in (q, k, v)]
    pt = torch.from_numpy(np.ascontiguousarray(page_table, np.int32)).to(dev)
    ln = torch.from_numpy(np.ascontiguousarray(lengths, np.int32)).to(dev)
    out = inkling.inkling_rpa(args[0], args[1], args[2], pt, ln, to_device_bf16(b, dev))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    exp = orc.inkling_rpa_reference(orc.bf16_to_f32(q), orc.bf16_to_f32(k), orc.bf16_to_f32(v),
                                    np.asarray(page_table), np.asarray(lengths), orc.bf16_to_f32(b))
    return got, exp


@pytest.mark.parametrize("seed", [0, 1, 7])
def test_contract_fixture(cuda, seed):
    _say(f"inkling-rpa contract fixture seed={seed}")
    got, exp = _run(cuda, *orc.inkling_rpa_inputs(seed))
    err = orc.errors(got, orc.bf16_round(exp))
    print(f"  max_abs={err['max_abs']:.3e} rel_l2={err['rel_l2']:.2e}")
    assert got.shape == (4, 4, 32) and err["finite"] and err["max_abs"] <= TOL, err


def test_uniform_keys_give_the_mean_of_v(cuda):
    """The reference's known-answer pattern (tests/test_workloads.py:42-60) with equal K/V heads:
    equal scores, zero bias -> every head outputs the mean of its kv head's first 5 V rows."""
    _say("inkling-rpa uniform keys")
    query = np.ones((1, 4, 8), np.float32)
    key_cache = np.ones((2, 4, 2, 8), np.float32)
    value_cache = np.arange(2 * 4 * 2 * 8, dtype=np.float32).reshape(2, 4, 2, 8) / 64.0
    got, _ = _run(cuda, query, key_cache, value_cache, np.array([[0, 1]], np.int32), np.array([5], np.int32),
                  np.zeros((4, 8), np.float32))
    rows = value_cache.reshape(-1, 2, 8)[:5]
    want = np.stack([rows[:, h // 2].mean(axis=0) for h in range(4)])
    assert np.allclose(got[0], want, atol=1e-2), (got[0], want)


def test_bias_selects_a_key_by_position(cuda):
    """A bias of +30 at one key position (0 elsewhere) and zero queries: the output is that key's V row."""
    _say("inkling-rpa bias by key position")
    rng = np.random.default_rng(5)
    key_cache = rng.normal(size=(8, 16, 2, 32)).astype(np.float32)
    value_cache = rng.normal(size=(8, 16, 2, 32)).astype(np.float32)
    page_table = np.array([[3, 1, 6, 0], [2, 7, 5, 4]], np.int32)
    lengths = np.array([50, 64], np.int32)
    bias = np.zeros((4, 64), np.float32)
    bias[:, 37] = 30.0
    got, exp = _run(cuda, np.zeros((2, 4, 32), np.float32), key_cache, value_cache, page_table, lengths, bias)
    for r in range(2):
        page, slot = page_table[r, 37 // 16], 37 % 16
        for h in range(4):
            want = orc.bf16_to_f32(orc.bf16_from_f32(value_cache[page, slot, h // 2]))
            assert np.allclose(got[r, h], want, atol=1e-2)
    assert orc.errors(got, orc.bf16_round(exp))["max_abs"] <= TOL


@pytest.mark.parametrize("hq,hkv,d,page", [(32, 8, 128, 64), (16, 4, 64, 16), (8, 8, 128, 32)])
def test_decode_shapes(cuda, hq, hkv, d, page):
    _say(f"inkling-rpa decode hq={hq} hkv={hkv} d={d} page={page}")
    rng = np.random.default_rng(hq * 7 + d + page)
    lengths = np.array([1, 31, 32, 33, 200, 517, 1000, 1500], np.int32)
    mp = int(-(-lengths.max() // page))
    pool = mp * len(lengths) + 5
    page_table = rng.permutation(pool)[: mp * len(lengths)].reshape(len(lengths), mp).astype(np.int32)
    query = rng.normal(size=(len(lengths), hq, d)).astype(np.float32)
    key_cache = rng.normal(size=(pool, page, hkv, d)).astype(np.float32)
    value_cache = rng.normal(size=(pool, page, hkv, d)).astype(np.float32)
    bias = rng.normal(scale=0.5, size=(hq, int(lengths.max()))).astype(np.float32)
    got, exp = _run(cuda, query, key_cache, value_cache, page_table, lengths, bias)
    err = orc.errors(got, orc.bf16_round(exp))
    print(f"  max_abs={err['max_abs']:.3e} rel_l2={err['rel_l2']:.2e}")
    assert err["finite"] and err["max_abs"] <= TOL, err


def test_checks_before_any_launch(cuda):
    q, k, v, pt, ln, b = orc.inkling_rpa_inputs(0)
    args = [to_device_bf16(orc.bf16_from_f32(x), cuda) for x in (q, k, v)]
    ptd = torch.from_numpy(pt).to(cuda)
    with pytest.raises(ValueError, match="cover every sequence length"):
        inkling.inkling_rpa(*args, ptd, torch.from_numpy(ln).to(cuda),
                            to_device_bf16(orc.bf16_from_f32(b[:, :100]), cuda))
    with pytest.raises(ValueError, match="one row per query head"):
        inkling.inkling_rpa(*args, ptd, torch.from_numpy(ln).to(cuda),
                            to_device_bf16(orc.bf16_from_f32(b[:3]), cuda))

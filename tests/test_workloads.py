"""The seeded benchmark configurations: determinism, shapes, page tables and byte counts."""

import math

import numpy as np
import pytest
import torch

from tpu_cake_amd import workloads as wl


def test_c1_is_seed_replayable_and_shaped():
    a = wl.make_config("c1", values="host")
    b = wl.make_config("c1", values="host")
    for f in ("q", "kv_pages", "kv_lens", "page_indices", "cu_q_lens", "num_seqs"):
        assert np.array_equal(getattr(a, f), getattr(b, f))
    assert a.q.shape == (4, 8, 128) and a.kv_pages.shape == (160, 16, 4, 128)
    assert a.page_indices.shape == (4, 32) and a.cu_q_lens.tolist() == [0, 1, 2, 3, 4]
    assert np.all((a.kv_lens >= 1) & (a.kv_lens <= 512))
    assert math.isclose(a.sm_scale, 1 / math.sqrt(128))


def _check_table(case):
    n = int(case.num_seqs[0])
    seen = set()
    for i in range(n):
        need = -(-int(case.kv_lens[i]) // case.page_size)
        row = case.page_indices[i]
        assert np.all(row[need:] == 0)  # padding slots hold 0, as upstream clamps them
        for p in row[:need]:
            assert 0 <= p < case.kv_pages.shape[0]
            assert p not in seen  # no page is shared within or across sequences
            seen.add(int(p))


@pytest.mark.parametrize("cfg", ["c1", "c2", "c3", "c5"])
def test_metadata_of_every_config(cfg, monkeypatch):
    # metadata only: skip the value draws by stubbing the normal generator
    # (keeps the pool's page count and page size, drops heads and dims)
    monkeypatch.setattr(wl, "_normal_bf16",
                        lambda rng, shape, *a, **k: np.zeros(tuple(shape[:2]) + (1,) * (len(shape) - 2), np.uint16))
    case = wl.make_config(cfg, values="host")
    _check_table(case)
    n = int(case.num_seqs[0])
    lens = case.kv_lens[:n]
    qlens = np.diff(case.cu_q_lens)
    if cfg == "c2":
        assert n == 64 and lens.min() >= 128 and lens.max() <= 8192 and np.all(qlens == 1)
        assert 1200 < np.median(lens) < 3500
    if cfg == "c3":
        assert n == 28 and np.all(qlens[:24] == 1) and np.all(qlens[24:] == 512)
        assert np.all(lens[:24] >= 512) and np.all(lens[24:] >= 512) and np.all(lens[24:] <= 3584 + 512)
    if cfg == "c5":
        assert n == 256 and lens.min() >= 16 and lens.max() <= 131072
    pool = case.kv_pages.shape[0]
    need = sum(-(-int(l) // case.page_size) for l in lens)
    assert pool == (160 if cfg == "c1" else math.ceil(1.25 * need))


def test_kv_read_bytes_formula():
    case = wl.make_custom(kv_lens=[10, 70], q_lens=[1, 1], num_q_heads=4, num_kv_heads=2, page_size=16,
                          values="host")
    assert case.kv_read_bytes() == 80 * 2 * 2 * 128 * 2
    f8 = wl.quantize_fp8(case)
    assert f8.kv_read_bytes() == 80 * 2 * 2 * 128 + (1 + 5) * 2 * 2 * 4


def test_fp8_quantisation_scales_and_codes():
    case = wl.make_custom(kv_lens=[40], q_lens=[1], num_q_heads=4, num_kv_heads=2, page_size=16, values="host")
    f8 = wl.quantize_fp8(case)
    src = torch.from_numpy(case.kv_pages.view(np.int16)).view(torch.bfloat16).float().numpy()
    P, S, C, D = src.shape
    amax = np.abs(src.reshape(P, S, 2, 2, D)).max(axis=(1, 4))
    np.testing.assert_allclose(f8.kv_scales, amax / 448.0, rtol=1e-6)
    deq = torch.from_numpy(f8.kv_pages).view(torch.float8_e4m3fn).float().numpy().reshape(P, S, 2, 2, D)
    assert np.abs(deq).max() <= 448.0
    err = np.abs(deq * f8.kv_scales[:, None, :, :, None] - src.reshape(P, S, 2, 2, D))
    assert err.max() <= amax.max() / 448.0 * 16  # half an e4m3 step at the top binade


def test_prefill_flops_count():
    case = wl.make_custom(kv_lens=[700, 5], q_lens=[100, 1], num_q_heads=8, num_kv_heads=2, page_size=64,
                          values="host")
    assert case.prefill_flops() == 4 * 8 * 128 * (100 * 600 + 100 * 101 // 2)

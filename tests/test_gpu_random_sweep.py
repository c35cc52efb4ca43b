"""GPU parity over random valid batches: KV modes (bf16, fp8, scalar K/V scales), page sizes
1..128, GQA groups 1..16 (including 3, 5, 6, 7), 1..12 kv heads (kv-head groups of 1..8 waves), decode rows and query chunks up to 80 tokens, sliding
window and soft cap, each against the oracle on the same inputs.

Bar per case: the reference's own gate, allclose(atol=rtol=0.02) (``src/tpu_cake/rpa_runner.py:105-122``),
and max-abs <= 2e-2 wherever |out| < 4 (from 4 up, one bf16 ulp is 2^-5 > 2e-2, so an absolute
bar below one ulp would reject any second rounding order).
"""

import numpy as np
import pytest
import torch

from oracle import rpa_oracle as orc
from tpu_cake_amd import ops
from tpu_cake_amd.workloads import make_custom

pytestmark = pytest.mark.gpu


def _random_case(rng):
    hkv = int(rng.choice([1, 2, 3, 4, 6, 8, 12]))
    g = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 16])) if hkv < 8 else int(rng.choice([1, 3, 4, 5, 8]))
    page = int(rng.choice([1, 8, 16, 24, 32, 64, 128]))
    kvl, ql = [], []
    for _ in range(int(rng.integers(1, 12))):
        L = int(rng.choice([rng.integers(1, 40), rng.integers(1, 600), rng.integers(500, 4000)]))
        kvl.append(L)
        ql.append(1 if rng.random() < 0.6 else int(rng.integers(1, min(L, 80) + 1)))
    mode = str(rng.choice(["bf16", "bf16", "fp8", "scaled"]))
    kw = {}
    if mode == "scaled":
        kw.update(k_scale=float(rng.uniform(0.5, 1.5)), v_scale=float(rng.uniform(0.5, 1.5)))
    if rng.random() < 0.2:
        kw["sliding_window"] = int(rng.integers(8, 300))
    if rng.random() < 0.15:
        kw["soft_cap"] = float(rng.uniform(2.0, 30.0))
    case = make_custom(kv_lens=kvl, q_lens=ql, num_q_heads=hkv * g, num_kv_heads=hkv, page_size=page,
                       seed=int(rng.integers(1 << 30)), kv_dtype="fp8" if mode == "fp8" else "bf16")
    return case, kw, f"hkv {hkv} g {g} page {page} kv {kvl} q {ql} mode {mode} kw {kw}"


@pytest.mark.parametrize("seed", [7, 11, 13])
def test_random_batches(cuda, seed):
    rng = np.random.default_rng(seed)
    for it in range(40):
        case, kw, desc = _random_case(rng)
        print(f"[case] sweep {seed}/{it}: {desc}", flush=True)
        out = ops.run_case(case, **kw)
        torch.cuda.synchronize()
        out = out.float().cpu().numpy()
        ref = orc.bf16_round(orc.ref_ragged_paged_attention(
            case.q, case.kv_pages, case.kv_lens, case.page_indices, case.cu_q_lens, case.num_seqs,
            sm_scale=case.sm_scale, kv_scales=case.kv_scales, kv_dtype=case.kv_dtype, probs_bf16=True, **kw))
        tv = ref.shape[0]
        got = out[:tv]
        assert np.all(np.isfinite(got)), desc
        assert np.allclose(got, ref, atol=0.02, rtol=0.02), desc
        small = np.abs(ref) < 4
        assert np.max(np.abs(got - ref)[small], initial=0.0) <= 2e-2, desc
        assert np.all(out[tv:] == 0.0), desc


def _prefill_heavy_case(rng):
    # mixed batches with enough prefill tiles that every CU holds a prefill-first workgroup (the
    # co-resident layout's fixed first tiles), over the layout's KV modes and page sizes
    hkv = int(rng.choice([4, 8, 12, 16]))
    g = int(rng.choice([1, 2, 4, 8])) if hkv <= 8 else int(rng.choice([1, 2, 4]))
    page = int(rng.choice([32, 64, 128]))
    kvl, ql = [], []
    for _ in range(int(rng.integers(2, 7))):  # prefill chunks over a prior
        q = int(rng.integers(200, 700))
        kvl.append(q + int(rng.integers(0, 2500)))
        ql.append(q)
    for _ in range(int(rng.integers(0, 6))):  # decode rows
        kvl.append(int(rng.integers(1, 5000)))
        ql.append(1)
    order = rng.permutation(len(kvl))
    kvl, ql = [kvl[i] for i in order], [ql[i] for i in order]
    mode = str(rng.choice(["bf16", "bf16", "fp8", "scaled"]))
    kw = {}
    if mode == "scaled":
        kw.update(k_scale=float(rng.uniform(0.5, 1.5)), v_scale=float(rng.uniform(0.5, 1.5)))
    if rng.random() < 0.25:
        kw["mask_value"] = float(rng.uniform(-8.0, -2.0))
    case = make_custom(kv_lens=kvl, q_lens=ql, num_q_heads=hkv * g, num_kv_heads=hkv, page_size=page,
                       seed=int(rng.integers(1 << 30)), kv_dtype="fp8" if mode == "fp8" else "bf16")
    return case, kw, f"hkv {hkv} g {g} page {page} kv {kvl} q {ql} mode {mode} kw {kw}"


def test_random_prefill_heavy_batches(cuda):
    rng = np.random.default_rng(2027)
    for it in range(10):
        case, kw, desc = _prefill_heavy_case(rng)
        print(f"[case] prefill-heavy sweep {it}: {desc}", flush=True)
        out = ops.run_case(case, **kw)
        torch.cuda.synchronize()
        out = out.float().cpu().numpy()
        ref = orc.bf16_round(orc.ref_ragged_paged_attention(
            case.q, case.kv_pages, case.kv_lens, case.page_indices, case.cu_q_lens, case.num_seqs,
            sm_scale=case.sm_scale, kv_scales=case.kv_scales, kv_dtype=case.kv_dtype, probs_bf16=True, **kw))
        tv = ref.shape[0]
        got = out[:tv]
        assert np.all(np.isfinite(got)), desc
        assert np.allclose(got, ref, atol=0.02, rtol=0.02), desc
        small = np.abs(ref) < 4
        assert np.max(np.abs(got - ref)[small], initial=0.0) <= 2e-2, desc

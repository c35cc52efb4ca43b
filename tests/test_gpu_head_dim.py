"""GPU parity for head dims other than 128 (the decode role's NW instantiation: narrower heads read
as 128-element rows, 256-dim heads as two 128-dim halves in paired waves): C2-shaped batches, fp8
pools, prefill rows, windows and soft caps, short pages, GQA groups and split row blocks, against
the CPU oracle at the bar of the 128-dim tests; the page-table gather bit-exact."""

import sys

import numpy as np
import pytest
import torch

from oracle import rpa_oracle as orc
from tpu_cake_amd import ops
from tpu_cake_amd.workloads import config_meta, make_custom

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _check(case, tol=TOL_BF16, **kw):
    out = ops.run_case(case, **kw)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert got.shape == case.q.shape
    ref = orc.ref_ragged_paged_attention(case.q, case.kv_pages, case.kv_lens, case.page_indices, case.cu_q_lens,
                                         case.num_seqs, sm_scale=case.sm_scale, kv_scales=case.kv_scales,
                                         kv_dtype=case.kv_dtype, **kw)
    tv = ref.shape[0]
    err = orc.errors(got[:tv], orc.bf16_round(ref))
    print(f"  max_abs={err['max_abs']:.3e} rel_l2={err['rel_l2']:.2e}", flush=True)
    assert err["finite"] and err["max_abs"] <= tol, err
    assert np.all(got[tv:] == 0.0)


def _c2_shaped(head_dim, kv_dtype="bf16", seed=7):
    m = config_meta("c2")
    return make_custom(kv_lens=m.kv_lens, q_lens=[1] * len(m.kv_lens), num_q_heads=32, num_kv_heads=8,
                       head_dim=head_dim, page_size=64, seed=seed, kv_dtype=kv_dtype)


@pytest.mark.parametrize("head_dim", [64, 96, 32, 256])
def test_c2_shaped_decode(cuda, head_dim):
    _say(f"C2-shaped decode, head_dim {head_dim}")
    _check(_c2_shaped(head_dim))


@pytest.mark.parametrize("head_dim", [64, 256])
def test_c2_shaped_fp8_decode(cuda, head_dim):
    # fp8 codes with per-(page, head) scales, against the same-codes oracle
    _say(f"C2-shaped fp8 decode, head_dim {head_dim}")
    _check(_c2_shaped(head_dim, kv_dtype="fp8", seed=9))


@pytest.mark.parametrize("head_dim,page", [(64, 64), (64, 16), (32, 16), (32, 64), (96, 24), (256, 64), (256, 16)])
def test_mixed_batch_prefill_rows(cuda, head_dim, page):
    # prefill rows run as causal stream-K row blocks at these head dims; page sizes that are not a
    # multiple of 32 take the operand-layout path
    _say(f"mixed batch, head_dim {head_dim}, page {page}")
    _check(make_custom(kv_lens=[700, 45, 1030, 9, 2100], q_lens=[1, 45, 130, 1, 300], num_q_heads=16,
                       num_kv_heads=4, head_dim=head_dim, page_size=page, seed=11 + head_dim + page))


@pytest.mark.parametrize("head_dim", [32, 64])
def test_scaled_pool_narrow_rows(cuda, head_dim):
    # scalar K/V scales (the scaled-bf16 mode) on whole-page units: the 32/64-element row loads
    _say(f"head_dim {head_dim}: k_scale 0.8, v_scale 1.3, page 64, prefill rows")
    case = make_custom(kv_lens=[2100, 70, 900, 4096], q_lens=[1, 40, 1, 1], num_q_heads=16, num_kv_heads=4,
                       head_dim=head_dim, page_size=64, seed=23 + head_dim)
    _check(case, k_scale=0.8, v_scale=1.3)


@pytest.mark.parametrize("head_dim", [64, 256])
def test_window_soft_cap_and_mask(cuda, head_dim):
    _say(f"head_dim {head_dim}: sliding window 512, soft cap 30, finite mask value")
    case = make_custom(kv_lens=[3000, 800, 5000, 64], q_lens=[1, 32, 1, 1], num_q_heads=32, num_kv_heads=8,
                       head_dim=head_dim, page_size=64, seed=13)
    _check(case, sliding_window=512, soft_cap=30.0)
    _check(case, mask_value=-2.5)


@pytest.mark.parametrize("head_dim,hq,hkv", [(64, 8, 2), (64, 12, 4), (64, 8, 8), (256, 8, 1), (256, 9, 3),
                                             (256, 16, 16)])
def test_gqa_groups(cuda, head_dim, hq, hkv):
    # 256: one kv head (a workgroup of its two halves), three (six halves), sixteen (two groups)
    _say(f"head_dim {head_dim}, Hq {hq} / Hkv {hkv}")
    _check(make_custom(kv_lens=[1500, 33, 4000, 700], q_lens=[1, 1, 3, 1], num_q_heads=hq, num_kv_heads=hkv,
                       head_dim=head_dim, page_size=32, seed=17 + hq))


@pytest.mark.parametrize("head_dim", [64, 256])
def test_long_sequence_split_over_many_workgroups(cuda, head_dim):
    # one 60000-key sequence over most of the grid (a heavy merge) beside short ones
    _say(f"head_dim {head_dim}, a 60000-key sequence")
    _check(make_custom(kv_lens=[60000, 40, 1, 3000], q_lens=[1, 1, 1, 1], num_q_heads=32, num_kv_heads=8,
                       head_dim=head_dim, page_size=64, seed=19))


@pytest.mark.parametrize("head_dim", [64, 256])
def test_gather_bit_exact(cuda, head_dim):
    _say(f"head_dim {head_dim} gather probe")
    case = make_custom(kv_lens=[100, 7, 300], q_lens=[1, 1, 1], num_q_heads=8, num_kv_heads=2, head_dim=head_dim,
                       page_size=16, seed=21)
    d = ops.case_to_device(case, "cuda")
    dense = ops.gather_kv(d["kv_pages"], d["kv_lens"], d["page_indices"], d["num_seqs"])
    torch.cuda.synchronize()
    got = dense.view(torch.int16).cpu().numpy().view(np.uint16)
    want = []
    for i in range(int(case.num_seqs[0])):
        k, v, _ = orc.gather_kv(case.kv_pages, case.page_indices, int(case.kv_lens[i]), i)
        both = np.empty((k.shape[0], 2 * k.shape[1], k.shape[2]), dtype=k.dtype)
        both[:, 0::2] = k
        both[:, 1::2] = v
        want.append(both)
    want = np.concatenate(want)
    assert got.shape == want.shape and np.array_equal(got, want)

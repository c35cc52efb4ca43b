"""Host-side operator checks that need no GPU: the reference's static/dynamic validation
messages (ragged_paged_attention.py:152-287) and loud failure on non-GPU tensors."""

import pytest
import torch

from tpu_cake_amd import ops


def _inputs(T=4, Hq=8, Hkv=2, D=128, P=10, S=16, N=3, PPS=4):
    return dict(
        q=torch.zeros(T, Hq, D, dtype=torch.bfloat16),
        kv_pages=torch.zeros(P, S, 2 * Hkv, D, dtype=torch.bfloat16),
        kv_lens=torch.tensor([5, 9, 20][:N], dtype=torch.int32),
        page_indices=torch.zeros(N, PPS, dtype=torch.int32),
        cu_q_lens=torch.tensor([0, 1, 2, 3][: N + 1], dtype=torch.int32),
        num_seqs=torch.tensor([N], dtype=torch.int32),
    )


def test_valid_inputs_pass_static_validation():
    ops.static_validate_inputs(**_inputs())


@pytest.mark.parametrize("mutate,msg", [
    (lambda d: d.update(num_seqs=torch.tensor([1, 1], dtype=torch.int32)), "num_seqs.shape"),
    (lambda d: d.update(kv_pages=torch.zeros(10, 16, 4, 64, dtype=torch.bfloat16)), "head_dim"),
    (lambda d: d.update(kv_lens=torch.zeros(4, dtype=torch.int32)), "kv_lens.shape"),
    (lambda d: d.update(cu_q_lens=torch.zeros(3, dtype=torch.int32)), "cu_q_lens.shape"),
    (lambda d: d.update(kv_lens=torch.zeros(3, dtype=torch.int64)), "int32"),
    (lambda d: d.update(q=torch.zeros(4, 6, 128, dtype=torch.bfloat16),
                        kv_pages=torch.zeros(10, 16, 8, 128, dtype=torch.bfloat16)), "divisible"),
])
def test_static_validation_messages(mutate, msg):
    d = _inputs()
    mutate(d)
    with pytest.raises(ValueError, match=msg):
        ops.static_validate_inputs(**d)


@pytest.mark.parametrize("kw,msg", [(dict(sliding_window=0), "sliding_window"), (dict(soft_cap=0.0), "soft_cap"),
                                    (dict(num_kv_pages_per_block=9), "num_kv_pages_per_block"),
                                    (dict(num_queries_per_block=0), "num_queries_per_block"),
                                    (dict(vmem_limit_bytes=0), "vmem_limit_bytes"),
                                    (dict(k_scale=1), "k_scale")])
def test_static_validation_of_knobs(kw, msg):
    with pytest.raises(ValueError, match=msg):
        ops.static_validate_inputs(**_inputs(), **kw)


def test_dynamic_validation_messages():
    d = _inputs()
    ops.dynamic_validate_inputs(**d)
    d2 = _inputs()
    d2["kv_lens"] = torch.tensor([5, 9, 100], dtype=torch.int32)
    with pytest.raises(ValueError, match="pages_per_seq"):
        ops.dynamic_validate_inputs(**d2)
    d3 = _inputs()
    d3["cu_q_lens"] = torch.tensor([0, 1, 2, 9], dtype=torch.int32)
    with pytest.raises(ValueError, match="Total q tokens"):
        ops.dynamic_validate_inputs(**d3)
    d4 = _inputs()
    d4["cu_q_lens"] = torch.tensor([0, 1, 2, 4], dtype=torch.int32)
    d4["kv_lens"] = torch.tensor([5, 9, 1], dtype=torch.int32)
    with pytest.raises(ValueError, match="q_len"):
        ops.dynamic_validate_inputs(**d4)


def test_operator_refuses_host_tensors():
    with pytest.raises(ValueError, match="GPU device"):
        ops.ragged_paged_attention(**_inputs(), sm_scale=0.1)


def test_no_cpu_fallback_without_library(monkeypatch, tmp_path):
    from tpu_cake_amd import _lib
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setenv("RPA_LIB", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.load()

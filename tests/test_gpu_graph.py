"""GPU: the operator captured into a HIP graph (ops.CapturedCall) and prepared once
(ops.PreparedCall), run over buffers whose values and metadata change in place -- every call
bitwise equal to an eager call on the same inputs, and within the oracle's tolerance.  Replays
are interleaved with the program's own eager work and synchronisations, as graph replays after the
first are where recorded memset nodes have gone wrong (the captured call records kernels only)."""

import sys

import numpy as np
import pytest
import torch

from oracle import rpa_oracle as orc
from tpu_cake_amd import ops
from tpu_cake_amd.workloads import make_config, make_custom

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _eager(d, case, out):
    return ops.ragged_paged_attention(d["q"], d["kv_pages"], d["kv_lens"], d["page_indices"], d["cu_q_lens"],
                                      d["num_seqs"], sm_scale=case.sm_scale, kv_scales=d.get("kv_scales"), out=out)


def _oracle_err(case, d, got):
    meta = {k: d[k].cpu().numpy() for k in ("kv_lens", "page_indices", "cu_q_lens", "num_seqs")}
    q = d["q"].view(torch.int16).cpu().numpy().view(np.uint16)
    kv = d["kv_pages"].view(torch.int16).cpu().numpy().view(np.uint16)
    ref = orc.ref_ragged_paged_attention(q, kv, meta["kv_lens"], meta["page_indices"], meta["cu_q_lens"],
                                         meta["num_seqs"], sm_scale=case.sm_scale)
    g = got.float().cpu().numpy()[: ref.shape[0]]
    return orc.errors(g, orc.bf16_round(ref))


@pytest.mark.parametrize("name", ["c1", "split"])
def test_captured_call_replays_match_eager(cuda, name):
    _say(f"graph replay {name}")
    if name == "c1":
        case = make_config("c1")
    else:  # long and short sequences over many workgroups: split row blocks, heavy merges, combine
        case = make_custom(kv_lens=[9000, 40, 1, 3000, 700, 64], q_lens=[1] * 6, num_q_heads=32, num_kv_heads=8,
                           page_size=64, seed=5)
    d = ops.case_to_device(case, "cuda")
    out_graph = torch.empty_like(d["q"])
    out_eager = torch.empty_like(d["q"])
    cc = ops.CapturedCall(d["q"], d["kv_pages"], d["kv_lens"], d["page_indices"], d["cu_q_lens"], d["num_seqs"],
                          sm_scale=case.sm_scale, out=out_graph)
    gen = torch.Generator(device="cuda").manual_seed(11)
    kv_lens0 = d["kv_lens"].clone()
    for r in range(5):
        # the loop's own work between replays: new values, and (from the third step) shorter
        # sequences -- the metadata of the same shapes
        d["q"].copy_(torch.randn(d["q"].shape, generator=gen, device="cuda").to(torch.bfloat16))
        if r >= 2:
            d["kv_lens"].copy_(torch.clamp(kv_lens0 - 37 * r, min=1))
        torch.cuda.synchronize()
        want = _eager(d, case, out_eager).clone()
        torch.cuda.synchronize()
        got = cc.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {r} differs from the eager call"
        if r in (0, 4):
            err = _oracle_err(case, d, got)
            print(f"  replay {r}: max_abs={err['max_abs']:.3e}", flush=True)
            assert err["finite"] and err["max_abs"] <= 2e-2, err


def test_captured_calls_layers_match_eager(cuda):
    """Four calls in one graph, as a model's decode step captures one call per layer: each layer
    has its own queries, K/V pool and output and all share the step's metadata tensors; the second
    and fourth layers carry an fp8 pool and a sliding window.  Every layer of every replay is
    bitwise equal to the same eager call."""
    _say("captured calls, 4 layers")
    case = make_custom(kv_lens=[700, 45, 1030, 9, 2100], q_lens=[1, 45, 30, 1, 64], num_q_heads=16,
                       num_kv_heads=4, page_size=64, seed=21)
    d = ops.case_to_device(case, "cuda")
    meta = (d["kv_lens"], d["page_indices"], d["cu_q_lens"], d["num_seqs"])
    gen = torch.Generator(device="cuda").manual_seed(17)
    layers = []
    for li in range(4):
        q = torch.randn(d["q"].shape, generator=gen, device="cuda").to(torch.bfloat16)
        if li % 2:
            kv = (torch.randn(d["kv_pages"].shape, generator=gen, device="cuda") * 4).to(torch.float8_e4m3fn)
            kw = dict(sm_scale=case.sm_scale, k_scale=0.5, v_scale=0.25, sliding_window=512)
        else:
            kv = torch.randn(d["kv_pages"].shape, generator=gen, device="cuda").to(torch.bfloat16)
            kw = dict(sm_scale=case.sm_scale)
        layers.append(((q, kv) + meta, kw))
    cc = ops.CapturedCalls(layers)
    kv_lens0 = d["kv_lens"].clone()
    q_lens = (d["cu_q_lens"][1:] - d["cu_q_lens"][:-1])[: kv_lens0.numel()].to(kv_lens0.dtype)
    for r in range(3):
        for (args, _) in layers:
            args[0].copy_(torch.randn(args[0].shape, generator=gen, device="cuda").to(torch.bfloat16))
        if r == 2:  # shorter sequences, still covering their query tokens
            d["kv_lens"].copy_(torch.maximum(kv_lens0 - 41, q_lens))
        torch.cuda.synchronize()
        wants = [ops.ragged_paged_attention(*args, **kw).clone() for args, kw in layers]
        torch.cuda.synchronize()
        gots = cc.replay()
        torch.cuda.synchronize()
        for li, (got, want) in enumerate(zip(gots, wants)):
            assert torch.equal(got, want), f"replay {r} layer {li} differs from the eager call"


def test_captured_calls_rejects_bad_calls(cuda):
    with pytest.raises(ValueError, match="no calls"):
        ops.CapturedCalls([])
    case = make_config("c1")
    d = ops.case_to_device(case, "cuda")
    with pytest.raises(ValueError, match="six positional"):
        ops.CapturedCalls([((d["q"], d["kv_pages"]), {})])


def test_captured_call_rejects_events(cuda):
    case = make_config("c1")
    d = ops.case_to_device(case, "cuda")
    with pytest.raises(ValueError, match="kernel_events"):
        ops.CapturedCall(d["q"], d["kv_pages"], d["kv_lens"], d["page_indices"], d["cu_q_lens"], d["num_seqs"],
                         sm_scale=case.sm_scale, kernel_events=(object(), object()))


@pytest.mark.parametrize("name", ["c1", "split"])
def test_prepared_call_matches_eager(cuda, name):
    """ops.PreparedCall over buffers whose values and metadata change in place: every call bitwise
    equal to an eager call on the same inputs."""
    _say(f"prepared call {name}")
    if name == "c1":
        case = make_config("c1")
    else:
        case = make_custom(kv_lens=[9000, 40, 1, 3000, 700, 64], q_lens=[1] * 6, num_q_heads=32, num_kv_heads=8,
                           page_size=64, seed=5)
    d = ops.case_to_device(case, "cuda")
    out_eager = torch.empty_like(d["q"])
    pc = ops.PreparedCall(d["q"], d["kv_pages"], d["kv_lens"], d["page_indices"], d["cu_q_lens"], d["num_seqs"],
                          sm_scale=case.sm_scale)
    gen = torch.Generator(device="cuda").manual_seed(13)
    kv_lens0 = d["kv_lens"].clone()
    for r in range(4):
        d["q"].copy_(torch.randn(d["q"].shape, generator=gen, device="cuda").to(torch.bfloat16))
        if r >= 2:
            d["kv_lens"].copy_(torch.clamp(kv_lens0 - 53 * r, min=1))
        want = _eager(d, case, out_eager).clone()
        got = pc()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {r} differs from the eager call"
        if r == 3:
            err = _oracle_err(case, d, got)
            assert err["finite"] and err["max_abs"] <= 2e-2, err


def test_prepared_call_rejects_unknown_keywords(cuda):
    case = make_config("c1")
    d = ops.case_to_device(case, "cuda")
    with pytest.raises(ValueError, match="kernel_events"):
        ops.PreparedCall(d["q"], d["kv_pages"], d["kv_lens"], d["page_indices"], d["cu_q_lens"], d["num_seqs"],
                         sm_scale=case.sm_scale, kernel_events=(object(), object()))

"""Fused Inkling decode on MI355X: one v3 RPA step (KV-cache write + relative-bias attention).

Mirrors the reference's fused plan (``src/tpu_cake/rpa_lowering.py``): ``preflight`` is its
``_preflight_decode_metadata`` (:71-128, same checks, same messages), ``run_preflighted``
(:275-288) runs it on host copies of the metadata before the kernel, and ``invoke`` (:232-273)
checks the eleven inputs' shapes and dtypes and runs the kernel.  The kernel semantics are those
the reference pins in ``inkling_fused_rpa_reference`` (``src/tpu_cake/workloads/inkling_rpa.py:
471-589``): write each sequence's new K/V token at position ``kv_len - 1`` of its pages, then
attend over the updated cache with scale ``1/D`` plus the relative-position bias; the cache is
updated in place and returned with the output (the reference aliases it).

Inputs, in the reference's order (all torch tensors on the GPU):
``queries`` bf16 [B, Hq, D], ``keys`` / ``values`` bf16 [B, Hkv, D], ``cache`` bf16
[P, S, 2*Hkv/packing, packing, W] (or [P, S, 2*Hkv, W]), ``kv_lengths`` i32 [B],
``page_indices`` i32 [entries], ``cu_q_lens`` i32 [B+1], ``cu_kv_lens`` i32 [B+1],
``distribution`` i32 [3], ``relative_states`` bf16 [B, Hq, R], ``relative_projection`` bf16 [R, E].
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib

INPUT_NAMES = ("queries", "keys", "values", "cache", "kv_lengths", "page_indices", "cu_q_lens", "cu_kv_lens",
               "distribution", "relative_states", "relative_projection")

_workspaces: dict = {}


def preflight(*inputs) -> None:
    """The reference's decode-metadata preflight (rpa_lowering.py:71-128) on host copies."""
    if len(inputs) != len(INPUT_NAMES):
        raise ValueError(f"fused RPA takes {len(INPUT_NAMES)} inputs, got {len(inputs)}")

    def host(x):
        return x.detach().cpu().numpy() if isinstance(x, torch.Tensor) else np.asarray(x)

    kv_lengths = host(inputs[4]).astype(np.int64)
    page_indices = host(inputs[5]).astype(np.int64).reshape(-1)
    cu_q = host(inputs[6]).astype(np.int64)
    cu_kv = host(inputs[7]).astype(np.int64)
    distribution = host(inputs[8]).astype(np.int64)
    cache_shape = tuple(inputs[3].shape)
    nseq = kv_lengths.shape[0]
    expected = np.full((3,), nseq, dtype=np.int64)
    if not np.array_equal(distribution, expected):
        raise ValueError("Inkling fused RPA adapter accepts decode-only distribution "
                         f"{tuple(expected)}, got {tuple(distribution)}")
    if not np.array_equal(cu_q, np.arange(nseq + 1, dtype=np.int64)):
        raise ValueError("Inkling fused RPA adapter requires one query token per sequence")
    if np.any(kv_lengths <= 0):
        raise ValueError("Inkling fused RPA requires positive KV lengths")
    page_size = cache_shape[1]
    if np.any(kv_lengths > cache_shape[0] * page_size):
        raise ValueError("fused RPA KV length exceeds total cache capacity")
    aligned = ((kv_lengths + page_size - 1) // page_size) * page_size
    expected_cu = np.concatenate((np.zeros((1,), np.int64), np.cumsum(aligned, dtype=np.int64)))
    if not np.array_equal(cu_kv, expected_cu):
        raise ValueError("fused RPA cumulative KV lengths must be page-aligned")
    required = int(expected_cu[-1]) // page_size
    if required > page_indices.size:
        raise ValueError("fused RPA page table cannot cover all KV lengths")
    used = page_indices[:required]
    if np.any(used < 0) or np.any(used >= cache_shape[0]):
        raise ValueError("fused RPA page index is outside the fused cache")
    page_sets = []
    for s in range(nseq):
        pages = page_indices[int(cu_kv[s]) // page_size: int(cu_kv[s + 1]) // page_size]
        if pages.size != np.unique(pages).size:
            raise ValueError("fused RPA page table aliases logical pages within one sequence")
        page_sets.append({int(x) for x in pages})
    writes = []
    for s, length in enumerate(kv_lengths):
        pos = int(length) - 1
        page = int(page_indices[int(cu_kv[s]) // page_size + pos // page_size])
        writes.append((page, pos % page_size))
    if len(writes) != len(set(writes)):
        raise ValueError("fused RPA decode updates collide in the physical cache")
    for w, (page, _) in enumerate(writes):
        for r, pages in enumerate(page_sets):
            if w != r and page in pages:
                raise ValueError("fused RPA active write page is shared across sequences")


def _check_signature(inputs):
    """Shapes and dtypes of the eleven inputs (rpa_lowering.py:213-226)."""
    if len(inputs) != len(INPUT_NAMES):
        raise ValueError(f"fused RPA takes {len(INPUT_NAMES)} inputs, got {len(inputs)}")
    for name, t in zip(INPUT_NAMES, inputs):
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError(f"{name} must be a CUDA (ROCm) tensor")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    q, k, v, cache = inputs[:4]
    for name, t in zip(("queries", "keys", "values", "cache", "relative_states", "relative_projection"),
                       (q, k, v, cache, inputs[9], inputs[10])):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bfloat16, got {t.dtype}")
    for name, t in zip(INPUT_NAMES[4:9], inputs[4:9]):
        if t.dtype != torch.int32:
            raise ValueError(f"{name} must be int32, got {t.dtype}")
    if q.dim() != 3 or k.dim() != 3 or v.shape != k.shape:
        raise ValueError("queries must be [B, Hq, D], keys and values [B, Hkv, D]")
    b, hq, d = q.shape
    if k.shape[0] != b or k.shape[2] != d or hq % k.shape[1]:
        raise ValueError(f"keys {tuple(k.shape)} do not match queries {tuple(q.shape)}")
    if cache.dim() == 5:
        rows = cache.shape[2] * cache.shape[3]
    elif cache.dim() == 4:
        rows = cache.shape[2]
    else:
        raise ValueError("cache must be [P, S, 2*Hkv/packing, packing, W] or [P, S, 2*Hkv, W]")
    if rows != 2 * k.shape[1]:
        raise ValueError(f"cache holds {rows} combined heads, expected {2 * k.shape[1]}")
    if cache.shape[-1] != 128 or d > 128:
        raise ValueError("cache width must be 128 and head_dim <= 128")
    if tuple(inputs[4].shape) != (b,) or tuple(inputs[6].shape) != (b + 1,) or tuple(inputs[7].shape) != (b + 1,):
        raise ValueError("kv_lengths must be [B], cu_q_lens and cu_kv_lens [B + 1]")
    if tuple(inputs[8].shape) != (3,):
        raise ValueError("distribution must be [3]")
    rs, rp = inputs[9], inputs[10]
    if rs.dim() != 3 or tuple(rs.shape[:2]) != (b, hq) or rp.dim() != 2 or rp.shape[0] != rs.shape[2]:
        raise ValueError("relative_states must be [B, Hq, R] and relative_projection [R, E]")


def invoke(*inputs, sm_scale: float | None = None, pages_per_seq: int | None = None,
           out: torch.Tensor | None = None):
    """Run the fused kernel on inputs that passed ``preflight``; returns (output, cache).

    ``pages_per_seq``: the largest ceil(kv_len / page_size) in the batch (computed from a host
    copy of kv_lengths when not given)."""
    _check_signature(inputs)
    q, k, v, cache = inputs[:4]
    b, hq, d = q.shape
    page_size = cache.shape[1]
    if pages_per_seq is None:
        pages_per_seq = int(((inputs[4].max().item() + page_size - 1) // page_size))
    rs, rp = inputs[9], inputs[10]
    shape = _lib.RpaFusedShape(num_seqs=b, num_q_heads=hq, num_kv_heads=k.shape[1], head_dim=d,
                               total_pages=cache.shape[0], page_size=page_size, cache_width=cache.shape[-1],
                               page_entries=inputs[5].numel(), pages_per_seq=max(1, pages_per_seq),
                               relative_dim=rs.shape[2], relative_extent=rp.shape[1])
    if sm_scale is None:
        sm_scale = 1.0 / d
    if out is None:
        out = torch.empty_like(q)
    lib = _lib.load()
    need = lib.rpa_fused_workspace_size(ctypes.byref(shape))
    if need == 0:
        _lib.check(-1)
    device = q.device
    stream = torch.cuda.current_stream(device).cuda_stream
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=device)
        _lib.check(lib.rpa_workspace_init(ws.data_ptr(), ws.numel(), stream))
        _workspaces[key] = ws
    with torch.cuda.device(device):
        rc = lib.rpa_inkling_fused_decode(
            ctypes.byref(shape), float(sm_scale), q.data_ptr(), k.data_ptr(), v.data_ptr(), cache.data_ptr(),
            inputs[4].data_ptr(), inputs[5].data_ptr(), inputs[6].data_ptr(), inputs[7].data_ptr(),
            inputs[8].data_ptr(), rs.data_ptr() if rs.numel() else None, rp.data_ptr() if rp.numel() else None,
            out.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc)
    return out, cache


def run_preflighted(*inputs, sm_scale: float | None = None, out: torch.Tensor | None = None):
    """preflight, then invoke (rpa_lowering.py:275-288): invalid metadata never reaches the kernel."""
    preflight(*inputs)
    page_size = inputs[3].shape[1]
    kv = inputs[4].detach().cpu().numpy().astype(np.int64)
    return invoke(*inputs, sm_scale=sm_scale, pages_per_seq=int(((kv + page_size - 1) // page_size).max()), out=out)


def read_error_word(device: torch.device | None = None) -> int:
    """The device-side error word of the fused workspace of the current stream."""
    device = device or torch.device("cuda", torch.cuda.current_device())
    stream = torch.cuda.current_stream(device).cuda_stream
    ws = _workspaces.get((device.index if device.index is not None else torch.cuda.current_device(), stream))
    if ws is None:
        return 0
    word = ctypes.c_int32(0)
    _lib.check(_lib.load().rpa_read_error_word(ws.data_ptr(), ws.numel(), ctypes.byref(word), stream))
    return int(word.value)

"""The v1 Inkling decode contract on MI355X (``experiment inkling-rpa``).

``inkling_rpa`` has the signature, argument meaning and ``ValueError`` checks of the reference's
``inkling_rpa_reference`` (``src/tpu_cake/workloads/inkling_rpa.py:37-73``): one query token per
sequence, separate key and value caches ``[P, S, Hkv, D]``, a ``[B, MP]`` page table, a bias
``[H, L]`` indexed by key position, scale ``1/D``; it returns ``[B, H, D]``.  The reference renders
this workload's experiment artifact (``src/tpu_cake/cli.py:667-676``, contract
``inkling_rpa.py:693-723``); here it runs through the C ABI entry ``rpa_inkling_decode`` (the
operator's kernels in relative-bias mode after one packing launch).

Inputs are torch tensors on the GPU: bf16 query, caches and bias (the contract's dtypes), int32
page table and lengths.  Key and value caches must have the same heads and head dim (the
contract's do), head_dim <= 128.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

_workspaces: dict = {}


def _check(query, key_cache, value_cache, page_table, sequence_lengths, bias):
    """The reference's checks (inkling_rpa.py:45-55, same messages), then this build's limits."""
    batch, query_heads, query_dimension = query.shape
    _, key_page_size, key_heads, key_dimension = key_cache.shape
    _, value_page_size, value_heads, value_dimension = value_cache.shape
    if key_page_size != value_page_size:
        raise ValueError("key and value caches must use the same page size")
    if query_dimension != key_dimension:
        raise ValueError("query and key head dimensions must match")
    if query_heads % key_heads or query_heads % value_heads:
        raise ValueError("query heads must divide evenly across key and value heads")
    if bias.shape[0] != query_heads:
        raise ValueError("relative bias must provide one row per query head")
    if key_cache.shape != value_cache.shape:
        raise ValueError("key and value caches must have the same shape on this backend")
    if query_dimension > 128:
        raise ValueError("head_dim must be <= 128")
    for name, t, dt in (("query", query, torch.bfloat16), ("key_cache", key_cache, torch.bfloat16),
                        ("value_cache", value_cache, torch.bfloat16), ("bias", bias, torch.bfloat16),
                        ("page_table", page_table, torch.int32), ("sequence_lengths", sequence_lengths, torch.int32)):
        if not isinstance(t, torch.Tensor) or not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous CUDA (ROCm) tensor")
        if t.dtype != dt:
            raise ValueError(f"{name} must be {dt}, got {t.dtype}")
    if page_table.dim() != 2 or page_table.shape[0] != batch or tuple(sequence_lengths.shape) != (batch,):
        raise ValueError("page_table must be [B, MP] and sequence_lengths [B]")
    if bias.dim() != 2:
        raise ValueError("bias must be [H, L]")
    lengths = sequence_lengths.detach().cpu()
    if bool((lengths < 1).any()):
        raise ValueError("sequence lengths must be positive")
    if int(lengths.max()) > bias.shape[1]:
        raise ValueError("relative bias must cover every sequence length")
    if int(lengths.max()) > page_table.shape[1] * key_page_size:
        raise ValueError("a sequence length exceeds its page table")


def inkling_rpa(query, key_cache, value_cache, page_table, sequence_lengths, bias, *, out=None):
    """Run the v1 Inkling decode on the GPU; returns bf16 ``[B, H, D]``."""
    _check(query, key_cache, value_cache, page_table, sequence_lengths, bias)
    b, h, d = query.shape
    shape = _lib.RpaInklingShape(num_seqs=b, num_q_heads=h, num_kv_heads=key_cache.shape[2], head_dim=d,
                                 total_pages=key_cache.shape[0], page_size=key_cache.shape[1],
                                 pages_per_seq=page_table.shape[1], bias_len=bias.shape[1])
    lib = _lib.load()
    need = lib.rpa_inkling_workspace_size(ctypes.byref(shape))
    if need == 0:
        _lib.check(-1)
    if out is None:
        out = torch.empty_like(query)
    device = query.device
    stream = torch.cuda.current_stream(device).cuda_stream
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=device)
        _lib.check(lib.rpa_workspace_init(ws.data_ptr(), ws.numel(), stream))
        _workspaces[key] = ws
    with torch.cuda.device(device):
        rc = lib.rpa_inkling_decode(ctypes.byref(shape), 1.0 / d, query.data_ptr(), key_cache.data_ptr(),
                                    value_cache.data_ptr(), page_table.data_ptr(), sequence_lengths.data_ptr(),
                                    bias.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc)
    return out

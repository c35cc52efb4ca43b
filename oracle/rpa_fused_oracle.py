"""CPU oracle for the fused Inkling decode (v3 RPA semantics) -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, as the checker; the product path
(``tpu_cake_amd``) never imports it.

A numpy restatement, written from the reference read as text (nothing of the
reference is imported), of:

* ``inkling_fused_rpa_inputs`` -- ``src/tpu_cake/workloads/inkling_rpa.py:413-468``
  (fixture: seeded bf16 tensors, the fixed 32-entry page list, page-aligned
  cumulative KV lengths, decode-only distribution);
* ``inkling_fused_rpa_reference`` -- ``inkling_rpa.py:471-589``: write each
  sequence's new K and V token at position ``kv_len - 1`` (page
  ``page_indices[cu_kv // S + pos // S]``, slot ``pos % S``, interleaved row
  ``2h`` / ``2h + 1``, zero-padded to the cache width), then attention over the
  updated cache with scale ``1/D`` and the relative-position bias
  ``relative_states[s] @ relative_projection[:, clip(L-1-l)]`` for distances
  below the projection width; fp32 softmax; (bf16 output, bf16 cache);
* ``FUSED_MUTATIONS`` -- ``FusedRpaOracleMutation``, ``inkling_rpa.py:404-410``;
* ``preflight_fused_decode`` -- ``_preflight_decode_metadata``,
  ``src/tpu_cake/rpa_lowering.py:71-128`` (same checks, same messages);
* ``fused_rpa_outputs_pass`` -- ``src/tpu_cake/rpa_runner.py:112-122``
  (allclose on the output, exact equality on the cache).

bf16 values are carried as uint16 bit patterns (``rpa_oracle.bf16_*``, RNE).

Pinning (``tests/test_fused_oracle.py``): the reference's own tests
``tests/test_rpa_oracle.py:10-39`` (seed replay, the page list's first six
entries, shapes and dtypes, cache changed, every mutation rejected by the
0.02/0.02 + exact-cache gate) and its preflight cases
``tests/test_rpa_lowering.py:604-653``; independently: the cache differs from
the input exactly at the written rows, which hold the new tokens zero-padded;
with zero relative states the output equals ``rpa_oracle.ref_ragged_paged_attention``
(separately pinned) at scale 1/D on the updated cache; a single-key sequence
returns its V row whatever the bias; equal keys give the softmax(bias)-weighted
mean of V (closed form).
"""

from __future__ import annotations

import math

import numpy as np

from oracle.rpa_oracle import bf16_from_f32, bf16_to_f32

FUSED_MUTATIONS = (
    "wrong_scale",
    "omit_relative_bias",
    "wrong_page_index",
    "ignore_page_indices",
    "swap_kv_interleave",
    "skip_cache_update",
)

# the fixture's page list (inkling_rpa.py:426-462)
FIXTURE_PAGES = (7, 2, 19, 4, 25, 1, 16, 9, 30, 12, 0, 5, 8, 11, 14, 17, 20, 23, 26, 29, 3, 6, 10, 13, 15,
                 18, 21, 22, 24, 27, 28, 31)


def inkling_fused_rpa_inputs(seed: int = 0) -> dict:
    """The reference fixture (inkling_rpa.py:413-468) as numpy; bf16 tensors as uint16 bits.

    Draw order and scales follow the reference: queries, keys, values (N(0,1)), cache (0.25),
    then relative states and projection (0.4), all float32 rounded to bf16 (RNE)."""
    rng = np.random.default_rng(seed)

    def bf16(shape, scale=1.0):
        return bf16_from_f32(rng.normal(scale=scale, size=shape).astype(np.float32))

    out = {
        "queries": bf16((4, 4, 32)),
        "keys": bf16((4, 2, 32)),
        "values": bf16((4, 2, 32)),
        "cache": bf16((32, 16, 2, 2, 128), scale=0.25),
        "kv_lengths": np.asarray((1, 17, 33, 49), dtype=np.int32),
        "page_indices": np.asarray(FIXTURE_PAGES, dtype=np.int32),
        "cu_q_lens": np.arange(5, dtype=np.int32),
        "cu_kv_lens": np.asarray((0, 16, 48, 96, 160), dtype=np.int32),
        "distribution": np.full((3,), 4, dtype=np.int32),
    }
    out["relative_states"] = bf16((4, 4, 16), scale=0.4)
    out["relative_projection"] = bf16((16, 128), scale=0.4)
    return out


def inkling_fused_rpa_reference(inp: dict, *, mutation: str | None = None):
    """(output bf16 bits [B, Hq, D], updated cache bf16 bits), inkling_rpa.py:471-589."""
    queries = bf16_to_f32(inp["queries"])
    keys = bf16_to_f32(inp["keys"])
    values = bf16_to_f32(inp["values"])
    cache = bf16_to_f32(inp["cache"]).copy()
    kv_lengths = np.asarray(inp["kv_lengths"], dtype=np.int32)
    page_indices = np.asarray(inp["page_indices"], dtype=np.int32).copy()
    cu_q = np.asarray(inp["cu_q_lens"], dtype=np.int32)
    cu_kv = np.asarray(inp["cu_kv_lens"], dtype=np.int32)
    distribution = np.asarray(inp["distribution"], dtype=np.int32)
    rel_states = bf16_to_f32(inp["relative_states"])
    rel_proj = bf16_to_f32(inp["relative_projection"])
    nseq = kv_lengths.shape[0]
    if not np.array_equal(distribution, np.full((3,), nseq, dtype=np.int32)):
        raise ValueError("fused RPA oracle requires a decode-only distribution")
    if not np.array_equal(cu_q, np.arange(nseq + 1, dtype=np.int32)):
        raise ValueError("fused RPA oracle requires one query token per sequence")
    if mutation == "ignore_page_indices":
        page_indices = np.arange(page_indices.size, dtype=np.int32)
    elif mutation == "wrong_page_index":
        page_indices[0] = (page_indices[0] + 1) % cache.shape[0]

    page_size, packing = cache.shape[1], cache.shape[3]
    key_slot, value_slot = (1, 0) if mutation == "swap_kv_interleave" else (0, 1)
    if mutation != "skip_cache_update":
        for s in range(nseq):
            pos = int(kv_lengths[s]) - 1
            page = page_indices[int(cu_kv[s]) // page_size + pos // page_size]
            slot = pos % page_size
            for h in range(keys.shape[1]):
                for kv_slot, src in ((key_slot, keys), (value_slot, values)):
                    row = 2 * h + kv_slot
                    dst = cache[page, slot, row // packing, row % packing]
                    dst.fill(0)
                    dst[: src.shape[-1]] = src[s, h]

    flat = cache.reshape(*cache.shape[:2], cache.shape[2] * packing, cache.shape[-1])
    d = queries.shape[-1]
    scale = 1.0 / math.sqrt(d) if mutation == "wrong_scale" else 1.0 / d
    extent = rel_proj.shape[1]
    group = queries.shape[1] // keys.shape[1]
    outputs = np.empty(queries.shape, dtype=np.float32)
    for s in range(nseq):
        length = int(kv_lengths[s])
        first = int(cu_kv[s]) // page_size
        pages = page_indices[first: first + math.ceil(length / page_size)]
        rows = flat[pages].reshape(-1, flat.shape[2], flat.shape[3])[:length]
        k = rows[:, key_slot::2, :d][:, : keys.shape[1]]
        v = rows[:, value_slot::2, :d][:, : values.shape[1]]
        # float32 products per (kv head, query head of its group): [Hkv, G, L]
        qg = queries[s].reshape(keys.shape[1], group, d)
        scores = np.matmul(qg, np.ascontiguousarray(k.transpose(1, 2, 0))).reshape(queries.shape[1], length)
        scores = scores * np.float32(scale)
        if mutation != "omit_relative_bias":
            dist = (length - 1) - np.arange(length, dtype=np.int32)
            proj = rel_proj[:, np.clip(dist, 0, extent - 1)]
            bias = np.matmul(rel_states[s], proj)
            scores = scores + np.where(dist[None] < extent, bias, np.float32(0.0))
        scores = scores - scores.max(axis=-1, keepdims=True)
        prob = np.exp(scores, dtype=np.float32)
        prob = prob / prob.sum(axis=-1, keepdims=True)
        pg = prob.reshape(keys.shape[1], group, length)
        outputs[s] = np.matmul(pg, np.ascontiguousarray(v.transpose(1, 0, 2))).reshape(queries.shape[1], d)
    return bf16_from_f32(outputs), bf16_from_f32(cache)


def preflight_fused_decode(inp: dict) -> None:
    """_preflight_decode_metadata (rpa_lowering.py:71-128): raises ValueError on bad metadata."""
    kv_lengths = np.asarray(inp["kv_lengths"], dtype=np.int64)
    page_indices = np.asarray(inp["page_indices"], dtype=np.int64)
    cu_q = np.asarray(inp["cu_q_lens"], dtype=np.int64)
    cu_kv = np.asarray(inp["cu_kv_lens"], dtype=np.int64)
    distribution = np.asarray(inp["distribution"], dtype=np.int64)
    cache_shape = np.shape(inp["cache"])
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


def fused_rpa_outputs_pass(actual, expected, *, output_atol: float = 0.02, output_rtol: float = 0.02) -> bool:
    """rpa_runner.py:112-122: output allclose, cache bit-exact (arrays as bf16 bits)."""
    return bool(np.allclose(bf16_to_f32(actual[0]), bf16_to_f32(expected[0]), atol=output_atol, rtol=output_rtol)
                and np.array_equal(actual[1], expected[1]))


def fused_inputs_like(seed: int, *, nseq: int, hq: int, hkv: int, d: int, page_size: int, pool_pages: int,
                      lengths, rel_dim: int, extent: int, dpad: int = 128, packing: int = 2) -> dict:
    """A larger fixture of the same contract (shapes of a real decode step): page-aligned
    cumulative KV lengths and a seeded permutation of the pool as the page list."""
    rng = np.random.default_rng(seed)
    lengths = np.asarray(lengths, dtype=np.int32)
    pages_needed = -(-lengths // page_size)
    cu_kv = np.concatenate(([0], np.cumsum(pages_needed * page_size))).astype(np.int32)
    perm = rng.permutation(pool_pages).astype(np.int32)
    assert int(pages_needed.sum()) <= pool_pages

    def bf16(shape, scale=1.0):
        return bf16_from_f32(rng.normal(scale=scale, size=shape).astype(np.float32))

    return {
        "queries": bf16((nseq, hq, d)),
        "keys": bf16((nseq, hkv, d)),
        "values": bf16((nseq, hkv, d)),
        "cache": bf16((pool_pages, page_size, 2 * hkv // packing, packing, dpad), scale=0.25),
        "kv_lengths": lengths,
        "page_indices": perm[: max(int(pages_needed.sum()), 1)].copy(),
        "cu_q_lens": np.arange(nseq + 1, dtype=np.int32),
        "cu_kv_lens": cu_kv,
        "distribution": np.full((3,), nseq, dtype=np.int32),
        "relative_states": bf16((nseq, hq, rel_dim), scale=0.4),
        "relative_projection": bf16((rel_dim, extent), scale=0.4),
    }

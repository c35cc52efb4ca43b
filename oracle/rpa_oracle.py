"""CPU oracle for ragged paged attention (RPA) -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.  The product
path (``tpu_cake_amd``) never imports it and has no CPU fallback.

It is a numpy restatement of the reference's RPA oracles, written from the
reference source read as text (nothing from the reference is imported):

* ``ref_ragged_paged_attention`` follows the upstream JAX oracle
  ``ecosystem/source/jax/ragged_paged_attention.py:73-148`` (mask value :32,
  validation :152-287).
* ``inkling_rpa_reference`` follows ``src/tpu_cake/workloads/inkling_rpa.py:37-73``.
* ``gather_kv`` restates the page-table gather both oracles share
  (``ragged_paged_attention.py:116-121``, ``inkling_rpa.py:62-64``).

Number formats are implemented here from their definitions (bf16 = top 16
bits of IEEE binary32 with round-to-nearest-even; fp8 e4m3 = OCP "E4M3FN",
bias 7, max 448, no infinities, NaN = S.1111.111), because ml_dtypes/JAX are
not installed.

Pinning (what checks each function; all in ``tests/test_oracle.py``):

* bf16 codec: exhaustive over all 2^16 patterns and 10^6 random floats
  against ``torch.bfloat16`` rounding.
* fp8 codec: exhaustive over the 256 codes (decode closed form, encode is the
  nearest-even representable value, saturation at 448).
* gather_kv: permutation invariance of the page pool, and equality with a
  dense contiguous layout built independently.
* ref_ragged_paged_attention: the reference's known answer
  (``tests/test_workloads.py:42-60``: uniform keys give the mean of V),
  kv_len == 1 gives the V row, float64 brute-force dense attention, textbook
  causal self-attention when q_len == kv_len, distinct-V GQA head mapping,
  and a mutation catalogue modelled on ``FusedRpaOracleMutation``
  (``inkling_rpa.py:404-410``) that each must fail the 2e-2 tolerance.
* inkling_rpa_reference: the reference's own known-answer test
  (``tests/test_workloads.py:42-60``) and determinism/finite checks.
"""

from __future__ import annotations

import math

import numpy as np

# ragged_paged_attention.py:32
DEFAULT_MASK_VALUE = -0.7 * float(np.finfo(np.float32).max)

FP8_E4M3_MAX = 448.0


# --------------------------------------------------------------------------
# Number formats
# --------------------------------------------------------------------------

def bf16_from_f32(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round-to-nearest-even.

    NaN inputs map to a quiet NaN.  Mirrors ``jnp.asarray(v, bfloat16)`` as
    used by the reference's input builders (``inkling_rpa.py:416-418``).
    """
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32)
    # no overflow for non-NaN patterns (at most 0xFF800000 + 0x8000); NaNs are replaced below
    rounding_bias = ((u >> np.uint32(16)) & np.uint32(1)) + np.uint32(0x7FFF)
    r = ((u + rounding_bias) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        r = np.where(nan, ((u >> np.uint32(16)).astype(np.uint16) | np.uint16(0x0040)), r).astype(np.uint16)
    return r


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> exact float32 values."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 value, returned as float32."""
    return bf16_to_f32(bf16_from_f32(x))


def _fp8_table() -> np.ndarray:
    codes = np.arange(256, dtype=np.uint32)
    sign = np.where(codes & 0x80, -1.0, 1.0)
    exp = (codes >> 3) & 0xF
    man = (codes & 0x7).astype(np.float64)
    val = np.where(exp == 0, man / 8.0 * 2.0 ** -6, (1.0 + man / 8.0) * 2.0 ** (exp.astype(np.float64) - 7.0))
    val = sign * val
    val[(codes & 0x7F) == 0x7F] = np.nan
    return val.astype(np.float32)


_FP8_DECODE = _fp8_table()


def fp8e4m3_to_f32(bits: np.ndarray) -> np.ndarray:
    """OCP fp8 e4m3 (E4M3FN) codes (uint8) -> float32."""
    return _FP8_DECODE[np.asarray(bits, dtype=np.uint8)]


def fp8e4m3_from_f32(x: np.ndarray) -> np.ndarray:
    """float32 -> OCP fp8 e4m3 codes, round-to-nearest-even, saturating at 448."""
    f = np.asarray(x, dtype=np.float32)
    finite = _FP8_DECODE[:0x7F].astype(np.float64)  # codes 0..126, increasing
    mag = np.minimum(np.abs(f).astype(np.float64), FP8_E4M3_MAX)
    hi = np.clip(np.searchsorted(finite, mag, side="left"), 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    d_hi = finite[hi] - mag
    d_lo = mag - finite[lo]
    # nearest representable magnitude; ties go to the even code (mantissa LSB 0)
    pick_lo = (hi != lo) & ((d_lo < d_hi) | ((d_lo == d_hi) & (lo % 2 == 0)))
    code = np.where(pick_lo, lo, hi).astype(np.uint16)
    code = code | (np.signbit(f).astype(np.uint16) << 7)
    code = np.where(np.isnan(f), np.uint16(0x7F), code)
    return code.astype(np.uint8)


# --------------------------------------------------------------------------
# Validation (ragged_paged_attention.py:152-287)
# --------------------------------------------------------------------------

def static_validate_inputs(q_shape, kv_shape, kv_lens, page_indices, cu_q_lens, num_seqs,
                           *, sliding_window=None, soft_cap=None) -> None:
    """Restates ``static_validate_inputs`` (ragged_paged_attention.py:216-287)."""
    _, num_q_heads, head_dim = q_shape
    _, _, num_combined, head_dim_k = kv_shape
    if num_combined % 2:
        raise ValueError(f"num_combined_kv_heads={num_combined} must be even")
    num_kv_heads = num_combined // 2
    max_num_seqs, _ = page_indices.shape
    if np.shape(num_seqs) != (1,):
        raise ValueError(f"num_seqs.shape={np.shape(num_seqs)} must be (1,)")
    if head_dim_k != head_dim:
        raise ValueError(f"Q head_dim {head_dim} must be the same as that of K/V {head_dim_k}.")
    if kv_lens.shape != (max_num_seqs,):
        raise ValueError(f"Expected kv_lens.shape={kv_lens.shape} to be ({max_num_seqs},)")
    if cu_q_lens.shape != (max_num_seqs + 1,):
        raise ValueError(f"Expected cu_q_lens.shape={cu_q_lens.shape} to be ({max_num_seqs + 1},)")
    if num_q_heads % num_kv_heads:
        raise ValueError(f"num_q_heads={num_q_heads} must be divisible by num_kv_heads={num_kv_heads}")
    if sliding_window is not None and sliding_window <= 0:
        raise ValueError(f"sliding_window={sliding_window} must be positive.")
    if soft_cap is not None and soft_cap == 0.0:
        raise ValueError(f"soft_cap={soft_cap} must not be 0.0.")


def dynamic_validate_inputs(num_tokens, page_size, kv_lens, page_indices, cu_q_lens, num_seqs) -> None:
    """Restates ``dynamic_validate_inputs`` (ragged_paged_attention.py:152-212)."""
    max_num_seqs, pages_per_seq = page_indices.shape
    n = int(np.asarray(num_seqs).reshape(-1)[0])
    if n > max_num_seqs:
        raise ValueError(f"num_seqs[0]={n} must be less or equal to max_num_seqs={max_num_seqs}")
    max_kv_len = int(np.max(kv_lens)) if kv_lens.size else 0
    min_pages = -(-max_kv_len // page_size)
    if pages_per_seq < min_pages:
        raise ValueError(f"pages_per_seq={pages_per_seq} must be greater or equal to min_pages_per_seq={min_pages}")
    if int(cu_q_lens[n]) > num_tokens:
        raise ValueError(f"Total q tokens {int(cu_q_lens[n])} must be less or equal to max_num_batched_tokens={num_tokens}.")
    for i in range(n):
        q_len = int(cu_q_lens[i + 1]) - int(cu_q_lens[i])
        if q_len > int(kv_lens[i]):
            raise ValueError(f"q_len={q_len} must be less or equal to kv_len={int(kv_lens[i])} at sequence {i}.")


# --------------------------------------------------------------------------
# Page-table gather
# --------------------------------------------------------------------------

def gather_kv(kv_pages: np.ndarray, page_indices: np.ndarray, kv_len: int, seq: int):
    """Dense K, V for one sequence, in logical token order.

    ``kv_pages`` is ``[P, S, 2*Hkv, D]`` (any element type); K of kv-head h is
    combined head 2h, V is 2h+1 (``ragged_paged_attention.py:116-121``).  Only
    logical pages ``< cdiv(kv_len, S)`` are touched (the reference reads
    ``page_indices[i]`` whole and slices ``[:kv_len]``; pages past the end
    never reach the result).  Returns ``(k, v, pages)`` with ``k, v`` shaped
    ``[kv_len, Hkv, D]``.
    """
    _, page_size, num_combined, head_dim = kv_pages.shape
    n_pages = -(-kv_len // page_size)
    pages = np.asarray(page_indices[seq, :n_pages], dtype=np.int64)
    block = kv_pages[pages].reshape(-1, num_combined, head_dim)[:kv_len]
    return block[:, 0::2, :], block[:, 1::2, :], pages


# --------------------------------------------------------------------------
# The upstream JAX oracle, restated
# --------------------------------------------------------------------------

def _decode_kv(x: np.ndarray, kv_dtype: str) -> np.ndarray:
    if kv_dtype == "bf16":
        return bf16_to_f32(x)
    if kv_dtype == "fp8":
        return fp8e4m3_to_f32(x)
    if kv_dtype == "f32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(kv_dtype)


def ref_ragged_paged_attention(
    q_bits: np.ndarray,            # uint16 bf16 [T, Hq, D]
    kv_pages: np.ndarray,          # uint16 bf16 | uint8 fp8 [P, S, 2*Hkv, D]
    kv_lens: np.ndarray,           # int32 [N_max]
    page_indices: np.ndarray,      # int32 [N_max, PPS]
    cu_q_lens: np.ndarray,         # int32 [N_max + 1]
    num_seqs: np.ndarray,          # int32 [1]
    *,
    sm_scale: float = 1.0,
    sliding_window: int | None = None,
    soft_cap: float | None = None,
    mask_value: float | None = DEFAULT_MASK_VALUE,
    k_scale: float | None = None,
    v_scale: float | None = None,
    kv_scales: np.ndarray | None = None,   # f32 [P, Hkv, 2] (build extension)
    kv_dtype: str = "bf16",
    probs_bf16: bool = True,
    _mutation: str | None = None,
) -> np.ndarray:
    """Restatement of ``ref_ragged_paged_attention`` (ragged_paged_attention.py:73-148).

    Returns float32 ``[cu_q_lens[num_seqs], Hq, D]`` holding the values the
    reference casts to the query dtype; round with ``bf16_from_f32`` for the
    bf16 output.  ``probs_bf16=True`` rounds softmax probabilities to bf16
    before the PV product (:144); ``False`` keeps float32 probabilities as the
    repo's numpy oracles do (``inkling_rpa.py:67-72``).  ``kv_scales`` is the
    per-(page, kv-head) K/V scale extension: dequantised K is
    ``bf16(f32(k) * kv_scales[page, h, 0])`` -- the reference's scalar
    ``k_scale`` formula (:124-129) applied per page.

    ``_mutation`` plants a known mistake (test use only).
    """
    if mask_value is None:
        mask_value = DEFAULT_MASK_VALUE
    T, num_q_heads, head_dim = q_bits.shape
    static_validate_inputs(q_bits.shape, kv_pages.shape, kv_lens, page_indices, cu_q_lens,
                           num_seqs, sliding_window=sliding_window, soft_cap=soft_cap)
    num_kv_heads = kv_pages.shape[2] // 2
    group = num_q_heads // num_kv_heads
    page_size = kv_pages.shape[1]
    q_all = bf16_to_f32(q_bits)
    pidx = np.asarray(page_indices)
    if _mutation == "ignore_page_indices":
        pidx = np.arange(pidx.size, dtype=np.int32).reshape(pidx.shape) % kv_pages.shape[0]
    elif _mutation == "wrong_page_index":
        pidx = pidx.copy()
        pidx[0, 0] = (pidx[0, 0] + 1) % kv_pages.shape[0]
    n = int(np.asarray(num_seqs).reshape(-1)[0])
    outs = []
    for i in range(n):
        q_start, q_end = int(cu_q_lens[i]), int(cu_q_lens[i + 1])
        q_len = q_end - q_start
        kv_len = int(kv_lens[i])
        q = q_all[q_start:q_end].astype(np.float64)
        k_raw, v_raw, pages = gather_kv(kv_pages, pidx, kv_len, i)
        if _mutation == "swap_kv_interleave":
            k_raw, v_raw = v_raw, k_raw
        k = _decode_kv(k_raw, kv_dtype)
        v = _decode_kv(v_raw, kv_dtype)
        if kv_scales is not None:
            tok_page = np.repeat(pages, page_size)[:kv_len]
            ks = kv_scales[tok_page, :, 0][:, :, None]
            vs = kv_scales[tok_page, :, 1][:, :, None]
            k = bf16_round((k * ks).astype(np.float32))
            v = bf16_round((v * vs).astype(np.float32))
        if k_scale is not None:
            k = bf16_round((k * np.float32(k_scale)).astype(np.float32))
        if v_scale is not None:
            v = bf16_round((v * np.float32(v_scale)).astype(np.float32))
        head_map = np.arange(num_q_heads) // group
        if _mutation == "wrong_gqa_map":
            head_map = np.arange(num_q_heads) % num_kv_heads
        # repeat(k, G, axis=1) then einsum("qhd,khd->hqk") (:130-133), computed per kv head as one
        # float64 matrix product over the q heads that map to it (the same sums, BLAS speed)
        kk = k.astype(np.float64)                    # [L, Hkv, D]
        vv = v.astype(np.float64)
        groups = [(hk, np.nonzero(head_map == hk)[0]) for hk in range(num_kv_heads)]
        attn = np.empty((num_q_heads, q_len, kv_len), dtype=np.float32)
        for hk, heads in groups:
            if heads.size:
                qh = q[:, heads, :].transpose(1, 0, 2).reshape(-1, head_dim)   # [g * q_len, D]
                attn[heads] = (qh @ kk[:, hk, :].T).reshape(heads.size, q_len, kv_len)
        scale = sm_scale if _mutation != "wrong_scale" else 1.0 / head_dim
        attn = (attn * np.float32(scale)).astype(np.float32)
        q_span = (kv_len - q_len) + np.arange(q_len)[None, :, None]
        kv_span = np.arange(kv_len)[None, None, :]
        mask = q_span < kv_span
        if _mutation == "no_causal_mask":
            mask = np.zeros_like(mask)
        if sliding_window is not None:
            mask = mask | (q_span - sliding_window >= kv_span)
        if soft_cap is not None:
            attn = (np.float32(soft_cap) * np.tanh(attn / np.float32(soft_cap))).astype(np.float32)
        attn = (attn + np.where(mask, np.float32(mask_value), np.float32(0.0))).astype(np.float32)
        attn = attn - attn.max(axis=-1, keepdims=True)
        e = np.exp(attn.astype(np.float64))
        probs = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
        if probs_bf16:
            probs = bf16_round(probs)
        out = np.empty((q_len, num_q_heads, head_dim), dtype=np.float32)
        for hk, heads in groups:   # einsum("hqk,khd->qhd") (:144-145), per kv head
            if heads.size:
                pv = probs[heads].astype(np.float64).reshape(-1, kv_len) @ vv[:, hk, :]
                out[:, heads, :] = pv.reshape(heads.size, q_len, head_dim).transpose(1, 0, 2)
        outs.append(out)
    if not outs:
        return np.zeros((0, num_q_heads, head_dim), dtype=np.float32)
    return np.concatenate(outs, axis=0)


def dense_attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, sm_scale: float,
                        causal_offset: int | None) -> np.ndarray:
    """Textbook softmax attention in float64 on dense arrays (brute force).

    ``q [Lq, Hq, D]``, ``k, v [L, Hq, D]`` (already GQA-expanded).  Query j sits
    at absolute position ``causal_offset + j`` when ``causal_offset`` is given.
    Written independently of ``ref_ragged_paged_attention`` (explicit loops
    over heads and rows) to check it.
    """
    Lq, H, _ = q.shape
    L = k.shape[0]
    out = np.zeros((Lq, H, v.shape[-1]), dtype=np.float64)
    for h in range(H):
        for j in range(Lq):
            limit = L if causal_offset is None else causal_offset + j + 1
            s = np.array([float(np.dot(q[j, h], k[t, h])) * sm_scale for t in range(limit)])
            w = np.exp(s - s.max())
            w /= w.sum()
            out[j, h] = (w[:, None] * v[:limit, h]).sum(axis=0)
    return out


# --------------------------------------------------------------------------
# The repo's Inkling numpy oracle (separate K/V caches + additive bias)
# --------------------------------------------------------------------------

def inkling_rpa_reference(query, key_cache, value_cache, page_table, sequence_lengths, bias):
    """Restates ``inkling_rpa_reference`` (src/tpu_cake/workloads/inkling_rpa.py:37-73).

    Scale is ``1/D`` (:68) and the output is float32 ``[B, Hq, Dv]``.
    """
    batch, query_heads, query_dim = query.shape
    _, page_size, key_heads, key_dim = key_cache.shape
    _, _, value_heads, value_dim = value_cache.shape
    if key_cache.shape[1] != value_cache.shape[1]:
        raise ValueError("key and value caches must use the same page size")
    if query_dim != key_dim:
        raise ValueError("query and key head dimensions must match")
    if query_heads % key_heads or query_heads % value_heads:
        raise ValueError("query heads must divide evenly across key and value heads")
    if bias.shape[0] != query_heads:
        raise ValueError("relative bias must provide one row per query head")
    kmap = np.arange(query_heads) // (query_heads // key_heads)
    vmap = np.arange(query_heads) // (query_heads // value_heads)
    out = np.empty((batch, query_heads, value_dim), dtype=np.float32)
    for r in range(batch):
        length = int(sequence_lengths[r])
        pages = page_table[r, : math.ceil(length / page_size)]
        keys = key_cache[pages].reshape(-1, key_heads, key_dim)[:length][:, kmap, :]
        values = value_cache[pages].reshape(-1, value_heads, value_dim)[:length][:, vmap, :]
        scores = np.einsum("hd,lhd->hl", query[r], keys, dtype=np.float32)
        scores = scores / query_dim + bias[:, :length]
        scores -= scores.max(axis=-1, keepdims=True)
        p = np.exp(scores)
        p /= p.sum(axis=-1, keepdims=True)
        out[r] = np.einsum("hl,lhd->hd", p, values, dtype=np.float32)
    return out


def inkling_rpa_inputs(seed: int = 0):
    """Seeded fixture of ``inkling_rpa_inputs`` (inkling_rpa.py:76-84), same draw order."""
    g = np.random.default_rng(seed)
    query = g.normal(size=(4, 4, 32)).astype(np.float32)
    key_cache = g.normal(size=(32, 16, 4, 32)).astype(np.float32)
    value_cache = g.normal(size=(32, 16, 4, 32)).astype(np.float32)
    page_table = np.arange(32, dtype=np.int32).reshape(4, 8)
    lengths = np.array([17, 33, 65, 127], dtype=np.int32)
    bias = g.normal(scale=0.05, size=(4, 128)).astype(np.float32)
    return query, key_cache, value_cache, page_table, lengths, bias


# --------------------------------------------------------------------------
# Error metrics (rpa_runner.py:105-122; rpa_surface_runner.py:394-411)
# --------------------------------------------------------------------------

def errors(actual: np.ndarray, expected: np.ndarray) -> dict:
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    diff = np.abs(a - e)
    denom = np.maximum(np.abs(e), np.finfo(np.float32).tiny)
    rel_l2 = float(np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-30))
    return {
        "max_abs": float(diff.max()) if diff.size else 0.0,
        "max_rel": float((diff / denom).max()) if diff.size else 0.0,
        "rel_l2": rel_l2,
        "finite": bool(np.isfinite(a).all()),
    }

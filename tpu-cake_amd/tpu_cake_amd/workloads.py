"""Seeded synthetic RPA workloads: the five MI355X benchmark configurations.

Each builder returns an :class:`RpaCase` of host numpy arrays in the
reference's operator layout (``ecosystem/source/jax/ragged_paged_attention.py:718-750``):

* ``q``            bf16 bits ``uint16 [T, Hq, D]``
* ``kv_pages``     bf16 bits ``uint16`` or fp8-e4m3 codes ``uint8`` ``[P, S, 2*Hkv, D]``;
                   K of kv-head h is combined head ``2h``, V is ``2h+1``
* ``kv_scales``    ``float32 [P, Hkv, 2]`` (K, V) for fp8 pools, else ``None``
* ``kv_lens``      ``int32 [N]``; ``page_indices`` ``int32 [N, PPS]``;
  ``cu_q_lens`` ``int32 [N+1]``; ``num_seqs`` ``int32 [1]``

Inputs follow the reference's recipe (``src/tpu_cake/workloads/inkling_rpa.py:413-418``):
N(0,1) float32 draws rounded to bf16 with round-to-nearest-even.  Lengths and
the page permutation come from ``numpy.random.default_rng(seed)`` in that
order.  Query and K/V values come from a second source chosen by ``values``:
``"host"`` continues the numpy generator (queries, then the pool), ``"cuda"``
draws them on the GPU with ``torch.Generator("cuda").manual_seed(seed * 16 + k)``
(k = 1 queries, k = 2 pool) -- the same distribution, fast for pools of
hundreds of MB.  Both are deterministic; ``"auto"`` picks ``"cuda"`` when a GPU
is present.  Logical page ``p`` of
sequence ``i`` is ``perm[offset_i + p]`` for ``p < cdiv(L_i, S)``; unused
page-table slots hold 0, as upstream clamps them (``ragged_paged_attention.py:53``).

Pinned choices the benchmark description leaves open:

* C2/C4 log-normal sigma = 0.5; C5 pool = 1.25x the pages in use (like C2).
* fp8 scales are separate for K and V: ``scale[p, h, c] = max|x| / 448`` over
  the (page, kv-head, K-or-V) tile of the bf16 source (1.0 for an all-zero tile).
* ``sm_scale = 1/sqrt(128)`` for every configuration.
"""

from __future__ import annotations

import dataclasses
import math

import numpy as np
import torch

LOGNORMAL_SIGMA = 0.5
POOL_FACTOR = 1.25
FP8_MAX = 448.0

CONFIG_SEEDS = {"c1": 97, "c2": 98, "c3": 99, "c4": 98, "c5": 101, "c3f": 99, "c5t": 101, "c2d64": 98, "c2d256": 98}

CONFIG_DESCRIPTIONS = {
    "c1": "tiny decode: 4 seqs x 1 token, kv_len U[1,512], Hq 8 / Hkv 2, D 128, page 16, 160-page pool",
    "c2": "GQA decode: 64 seqs x 1 token, kv_len lognormal(median 2048, sigma 0.5) clip 128-8192, Hq 32 / Hkv 8, D 128, page 64",
    "c3": "mixed: 24 decode rows (kv_len U[512,8192]) + 4 causal prefill chunks of 512 over prior U[0,3584], Hq 32 / Hkv 8, page 64",
    "c4": "fp8-e4m3 KV decode: C2 shapes, per-(page, kv head) K and V scales = max|x|/448",
    "c5": "heavy-tail decode: 256 seqs x 1 token, kv_len 16*(1+Lomax(1.2)) clip 16-131072, Hq 64 / Hkv 8, D 128, page 64",
    # the two below are this build's measurement workloads beside BASELINE's five
    "c3f": "C3's mixed batch (24 decode rows + 4 prefill chunks of 512) over an fp8-e4m3 pool with per-(page, kv head) K and V scales = max|x|/448",
    "c5t": "C5 with its first sequence at the clip, 131072 keys (the heavy tail's worst case)",
    "c2d64": "C2's batch with head_dim 64 (the narrow decode instantiation)",
    "c2d256": "C2's batch with head_dim 256 (two 128-dim halves per kv head)",
}


@dataclasses.dataclass
class RpaCase:
    name: str
    q: np.ndarray
    kv_pages: np.ndarray
    kv_lens: np.ndarray
    page_indices: np.ndarray
    cu_q_lens: np.ndarray
    num_seqs: np.ndarray
    sm_scale: float
    kv_dtype: str = "bf16"
    kv_scales: np.ndarray | None = None
    kv_source: np.ndarray | None = None  # bf16 pool the fp8 pool was quantised from

    @property
    def num_q_heads(self) -> int:
        return int(self.q.shape[1])

    @property
    def num_kv_heads(self) -> int:
        return int(self.kv_pages.shape[2] // 2)

    @property
    def head_dim(self) -> int:
        return int(self.q.shape[2])

    @property
    def page_size(self) -> int:
        return int(self.kv_pages.shape[1])

    @property
    def q_lens(self) -> np.ndarray:
        n = int(self.num_seqs[0])
        return np.diff(self.cu_q_lens[: n + 1]).astype(np.int64)

    def work(self, sliding_window: int | None = None):
        """The call's algorithmic work (``tpu_cake_amd.cost_model.rpa_work``)."""
        from .cost_model import rpa_work

        n = int(self.num_seqs[0])
        return rpa_work(self.kv_lens[:n], self.q_lens, num_q_heads=self.num_q_heads,
                        num_kv_heads=self.num_kv_heads, head_dim=self.head_dim, page_size=self.page_size,
                        kv_dtype=self.kv_dtype, sliding_window=sliding_window)

    def kv_read_bytes(self, sliding_window: int | None = None) -> int:
        """Algorithmic KV bytes one call must read: every key some query row sees, K and V of every
        kv head (sum(L) * Hkv * 2 * D * elem without a window), plus the fp8 scales of those pages."""
        w = self.work(sliding_window)
        return w.kv_read_bytes + w.scale_bytes

    def prefill_flops(self, sliding_window: int | None = None) -> int:
        """Causal QK^T + PV flops of rows with q_len > 1: 4*Hq*D*sum(visible keys)."""
        return self.work(sliding_window).prefill_flops


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (via torch's cast)."""
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _page_table(rng, kv_lens, page_size, pool_pages, pages_per_seq):
    need = -(-kv_lens.astype(np.int64) // page_size)
    total = int(need.sum())
    if total > pool_pages:
        raise ValueError(f"pool of {pool_pages} pages cannot hold {total} pages")
    perm = rng.permutation(pool_pages).astype(np.int32)
    table = np.zeros((len(kv_lens), pages_per_seq), dtype=np.int32)
    off = 0
    for i, n in enumerate(need):
        table[i, :n] = perm[off: off + n]
        off += int(n)
    return table


def _normal_bf16(rng, shape, values: str = "host", seed: int = 0, stream: int = 0) -> np.ndarray:
    if values == "cuda":
        g = torch.Generator(device="cuda").manual_seed(int(seed) * 16 + stream)
        x = torch.randn(shape, generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
        return x.view(torch.int16).cpu().numpy().view(np.uint16)
    return f32_to_bf16_bits(rng.standard_normal(size=shape, dtype=np.float32))


def _resolve_values(values: str) -> str:
    if values == "auto":
        return "cuda" if torch.cuda.is_available() else "host"
    if values not in ("host", "cuda"):
        raise ValueError(f"values must be 'auto', 'host' or 'cuda', got {values!r}")
    return values


def build_case(name: str, *, kv_lens, q_lens, num_q_heads, num_kv_heads, head_dim, page_size,
               pool_pages, pages_per_seq, rng, sm_scale=None, values="host", seed=0) -> RpaCase:
    kv_lens = np.asarray(kv_lens, dtype=np.int32)
    q_lens = np.asarray(q_lens, dtype=np.int32)
    table = _page_table(rng, kv_lens, page_size, pool_pages, pages_per_seq)
    cu = np.zeros(len(kv_lens) + 1, dtype=np.int32)
    cu[1:] = np.cumsum(q_lens)
    T = int(cu[-1])
    q = _normal_bf16(rng, (T, num_q_heads, head_dim), values, seed, 1)
    kv = _normal_bf16(rng, (pool_pages, page_size, 2 * num_kv_heads, head_dim), values, seed, 2)
    return RpaCase(
        name=name, q=q, kv_pages=kv, kv_lens=kv_lens, page_indices=table, cu_q_lens=cu,
        num_seqs=np.array([len(kv_lens)], dtype=np.int32),
        sm_scale=float(sm_scale if sm_scale is not None else 1.0 / math.sqrt(head_dim)),
    )


def quantize_fp8(case: RpaCase) -> RpaCase:
    """fp8-e4m3 pool + per-(page, kv-head, K|V) scales from a bf16 case."""
    P, S, C, D = case.kv_pages.shape
    Hkv = C // 2
    dev = "cuda" if torch.cuda.is_available() else "cpu"
    src = torch.from_numpy(case.kv_pages.view(np.int16)).view(torch.bfloat16).to(dev)
    x = src.float().view(P, S, Hkv, 2, D)
    amax = x.abs().amax(dim=(1, 4))  # [P, Hkv, 2]
    scale = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    q = (x / scale.view(P, 1, Hkv, 2, 1)).clamp_(-FP8_MAX, FP8_MAX)
    codes = q.to(torch.float8_e4m3fn).view(torch.uint8).view(P, S, C, D).cpu().numpy()
    return dataclasses.replace(case, kv_pages=codes, kv_dtype="fp8",
                               kv_scales=scale.cpu().numpy().astype(np.float32),
                               kv_source=case.kv_pages)


@dataclasses.dataclass(frozen=True)
class ConfigMeta:
    """Shapes and metadata of a benchmark configuration (no values): what a contract names."""
    name: str
    kv_lens: np.ndarray
    q_lens: np.ndarray
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    page_size: int
    pool_pages: int
    pages_per_seq: int
    kv_dtype: str = "bf16"

    @property
    def num_tokens(self) -> int:
        return int(np.sum(self.q_lens))

    @property
    def num_seqs(self) -> int:
        return len(self.kv_lens)

    def work(self, sliding_window: int | None = None):
        from .cost_model import rpa_work

        return rpa_work(self.kv_lens, self.q_lens, num_q_heads=self.num_q_heads, num_kv_heads=self.num_kv_heads,
                        head_dim=self.head_dim, page_size=self.page_size, kv_dtype=self.kv_dtype,
                        sliding_window=sliding_window)

    def kv_read_bytes(self, sliding_window: int | None = None) -> int:
        """sum(L) * Hkv * 2 * D * elem (+ the fp8 pool's per-(page, head) K and V scales)."""
        w = self.work(sliding_window)
        return w.kv_read_bytes + w.scale_bytes

    def prefill_flops(self, sliding_window: int | None = None) -> int:
        """Causal QK^T + PV flops of rows with q_len > 1: 4*Hq*D*sum(visible keys)."""
        return self.work(sliding_window).prefill_flops


def _config_meta(cfg: str, rng) -> ConfigMeta:
    """The lengths and shapes of ``cfg``, drawn from ``rng`` (the first draws of make_config)."""
    if cfg == "c1":
        lens = rng.integers(1, 512, size=4, endpoint=True)
        return ConfigMeta("c1", lens, np.ones(4, np.int64), 8, 2, 128, 16, 160, 32)
    if cfg in ("c2", "c4"):
        z = rng.standard_normal(64)
        lens = np.clip(np.rint(np.exp(math.log(2048.0) + LOGNORMAL_SIGMA * z)), 128, 8192).astype(np.int64)
        pages = int(np.sum(-(-lens // 64)))
        return ConfigMeta(cfg, lens, np.ones(64, np.int64), 32, 8, 128, 64, math.ceil(POOL_FACTOR * pages), 128,
                          "fp8" if cfg == "c4" else "bf16")
    if cfg == "c3":
        dec = rng.integers(512, 8192, size=24, endpoint=True)
        prior = rng.integers(0, 3584, size=4, endpoint=True)
        lens = np.concatenate([dec, prior + 512])
        qls = np.concatenate([np.ones(24, dtype=np.int64), np.full(4, 512)])
        pages = int(np.sum(-(-lens // 64)))
        return ConfigMeta("c3", lens, qls, 32, 8, 128, 64, math.ceil(POOL_FACTOR * pages), 128)
    if cfg == "c3f":
        m = _config_meta("c3", rng)
        return dataclasses.replace(m, name="c3f", kv_dtype="fp8")
    if cfg in ("c2d64", "c2d256"):
        m = _config_meta("c2", rng)
        return dataclasses.replace(m, name=cfg, head_dim=64 if cfg == "c2d64" else 256)
    if cfg in ("c5", "c5t"):
        lens = np.clip(np.floor(16.0 * (1.0 + rng.pareto(1.2, size=256))), 16, 131072).astype(np.int64)
        if cfg == "c5t":
            lens[0] = 131072
        pages = int(np.sum(-(-lens // 64)))
        return ConfigMeta(cfg, lens, np.ones(256, np.int64), 64, 8, 128, 64, math.ceil(POOL_FACTOR * pages), 2048)
    raise ValueError(f"unknown config {cfg!r}; expected one of {sorted(CONFIG_SEEDS)}")


def config_meta(cfg: str, seed: int | None = None) -> ConfigMeta:
    """Shapes and lengths of configuration ``cfg`` (the same draws as make_config), no values."""
    cfg = cfg.lower()
    if cfg not in CONFIG_SEEDS:
        raise ValueError(f"unknown config {cfg!r}; expected one of {sorted(CONFIG_SEEDS)}")
    return _config_meta(cfg, np.random.default_rng(CONFIG_SEEDS[cfg] if seed is None else seed))


def make_config(cfg: str, seed: int | None = None, values: str = "auto") -> RpaCase:
    """Build one of the benchmark configurations ``c1`` .. ``c5`` (or ``c3f`` / ``c5t``)."""
    cfg = cfg.lower()
    if cfg not in CONFIG_SEEDS:
        raise ValueError(f"unknown config {cfg!r}; expected one of {sorted(CONFIG_SEEDS)}")
    if seed is None:
        seed = CONFIG_SEEDS[cfg]
    rng = np.random.default_rng(seed)
    m = _config_meta(cfg, rng)
    case = build_case(cfg, kv_lens=m.kv_lens, q_lens=m.q_lens, num_q_heads=m.num_q_heads,
                      num_kv_heads=m.num_kv_heads, head_dim=m.head_dim, page_size=m.page_size,
                      pool_pages=m.pool_pages, pages_per_seq=m.pages_per_seq, rng=rng,
                      values=_resolve_values(values), seed=seed)
    return quantize_fp8(case) if cfg in ("c4", "c3f") else case


def make_custom(*, kv_lens, q_lens, num_q_heads, num_kv_heads, head_dim=128, page_size=16,
                pool_factor=1.25, pages_per_seq=None, seed=0, sm_scale=None, max_num_seqs=None,
                num_tokens=None, kv_dtype="bf16", values="auto") -> RpaCase:
    """Small ad-hoc case for tests: explicit lengths, optional padding of N_max / T."""
    rng = np.random.default_rng(seed)
    kv_lens = np.asarray(kv_lens, dtype=np.int64)
    need = int(np.sum(-(-kv_lens // page_size)))
    pps = pages_per_seq or max(1, int(-(-max(int(kv_lens.max(initial=0)), 1) // page_size)))
    case = build_case("custom", kv_lens=kv_lens, q_lens=q_lens, num_q_heads=num_q_heads,
                      num_kv_heads=num_kv_heads, head_dim=head_dim, page_size=page_size,
                      pool_pages=max(1, math.ceil(pool_factor * need)), pages_per_seq=pps, rng=rng,
                      sm_scale=sm_scale, values=_resolve_values(values), seed=seed)
    n = len(kv_lens)
    if max_num_seqs is not None and max_num_seqs > n:
        pad = max_num_seqs - n
        case.kv_lens = np.concatenate([case.kv_lens, np.zeros(pad, np.int32)])
        case.page_indices = np.concatenate([case.page_indices, np.zeros((pad, pps), np.int32)])
        case.cu_q_lens = np.concatenate([case.cu_q_lens, np.full(pad, case.cu_q_lens[-1], np.int32)])
    if num_tokens is not None and num_tokens > case.q.shape[0]:
        extra = _normal_bf16(rng, (num_tokens - case.q.shape[0],) + case.q.shape[1:])
        case.q = np.concatenate([case.q, extra])
    if kv_dtype == "fp8":
        case = quantize_fp8(case)
    return case


# ---------------------------------------------------------------------------------------------
# the fused Inkling decode step (v3 contract, src/tpu_cake/workloads/inkling_rpa.py:413-589)
# ---------------------------------------------------------------------------------------------
FUSED_DESCRIPTION = ("inkling fused decode: C2 lengths (64 seqs, lognormal median 2048) incl. the new token, "
                     "Hq 32 / Hkv 8, D 128, page 64, relative bias R 16 / E 512, cache write + attention")


@dataclasses.dataclass
class FusedCase:
    """Inputs of one fused decode step in the reference's order (``fused.INPUT_NAMES``): bf16
    tensors as uint16 bits, metadata int32."""
    arrays: dict
    sm_scale: float

    def kv_read_bytes(self) -> int:
        n_kv = self.arrays["keys"].shape[1]
        return int(self.arrays["kv_lengths"].astype(np.int64).sum()) * n_kv * 2 * 128 * 2


def make_fused_case(seed: int = 102, *, nseq: int = 64, num_q_heads: int = 32, num_kv_heads: int = 8,
                    head_dim: int = 128, page_size: int = 64, relative_dim: int = 16, relative_extent: int = 512,
                    values: str = "auto", lengths=None) -> FusedCase:
    """A fused decode step at Inkling decode shapes: page-aligned cumulative KV lengths and a
    seeded permutation of a 1.25x pool as the flat page list (each sequence's pages consecutive
    in it), N(0,1) queries / new K,V, N(0, 0.25) cache, N(0, 0.4) relative tensors (the
    reference fixture's scales, inkling_rpa.py:413-424)."""
    rng = np.random.default_rng(seed)
    if lengths is None:
        z = rng.standard_normal(nseq)
        lengths = np.clip(np.round(np.exp(math.log(2048.0) + LOGNORMAL_SIGMA * z)), 128, 8192)
    lengths = np.asarray(lengths, dtype=np.int32)
    pages_needed = -(-lengths // page_size)
    pool = int(math.ceil(POOL_FACTOR * int(pages_needed.sum())))
    perm = rng.permutation(pool).astype(np.int32)
    cu_kv = np.concatenate(([0], np.cumsum(pages_needed * page_size))).astype(np.int32)
    v = _resolve_values(values)

    def normal(shape, scale, stream):  # N(0, scale^2) float32 rounded to bf16
        if v == "cuda":
            g = torch.Generator(device="cuda").manual_seed(int(seed) * 16 + stream)
            x = torch.randn(shape, generator=g, device="cuda", dtype=torch.float32) * scale
            return x.to(torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
        return f32_to_bf16_bits(rng.standard_normal(size=shape, dtype=np.float32) * np.float32(scale))

    arrays = {
        "queries": normal((nseq, num_q_heads, head_dim), 1.0, 3),
        "keys": normal((nseq, num_kv_heads, head_dim), 1.0, 4),
        "values": normal((nseq, num_kv_heads, head_dim), 1.0, 5),
        "cache": normal((pool, page_size, 2 * num_kv_heads, 128), 0.25, 6),
        "kv_lengths": lengths,
        "page_indices": perm[: int(pages_needed.sum())].copy(),
        "cu_q_lens": np.arange(nseq + 1, dtype=np.int32),
        "cu_kv_lens": cu_kv,
        "distribution": np.full((3,), nseq, dtype=np.int32),
        "relative_states": normal((nseq, num_q_heads, relative_dim), 0.4, 7),
        "relative_projection": normal((relative_dim, relative_extent), 0.4, 8),
    }
    return FusedCase(arrays=arrays, sm_scale=1.0 / head_dim)


def fused_lengths(seed: int = 102, nseq: int = 64) -> np.ndarray:
    """The kv lengths make_fused_case draws for ``seed`` (its first draws), without the arrays."""
    z = np.random.default_rng(seed).standard_normal(nseq)
    return np.clip(np.round(np.exp(math.log(2048.0) + LOGNORMAL_SIGMA * z)), 128, 8192).astype(np.int64)


def make_fused_meta(seed: int = 102, *, nseq: int = 64, num_q_heads: int = 32, num_kv_heads: int = 8) -> dict:
    """Byte counts of the fused decode step of make_fused_case(seed) (KV read, Q, O and the new
    K/V rows written), from its lengths alone."""
    lens = fused_lengths(seed, nseq)
    kv = int(lens.sum()) * num_kv_heads * 2 * 128 * 2
    qo = 2 * nseq * num_q_heads * 128 * 2
    new_rows = 2 * nseq * num_kv_heads * 128 * 2 * 2  # keys and values, read and written
    return {"kv_read_bytes": kv, "moved_bytes": kv + qo + new_rows}


WINDOWED_CONFIGS = {"c2w": ("c2", 512)}


def make_config_meta_for(name: str):
    """(ConfigMeta, sliding window or None) of a benchmark configuration, including the windowed
    ones (``c2w``: C2 with a 512-key sliding window)."""
    base, window = WINDOWED_CONFIGS.get(name, (name, None))
    return config_meta(base), window

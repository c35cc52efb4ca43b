"""The RPA operator on MI355X: the reference's Python surface over ``librpa.so``.

``ragged_paged_attention`` keeps the signature and error behaviour of the
upstream JAX operator (``ecosystem/source/jax/ragged_paged_attention.py:718-899``):
the same positional tensors, the same keyword knobs, ``ValueError`` with the
reference's messages from ``static_validate_inputs`` (:216-287) before any
launch, and a fresh output shaped like ``q``.  Tensors are torch tensors on the
GPU (torch is only the allocator); the work is two HIP kernels launched through
the C ABI on torch's current stream.  The Pallas block-size knobs
(``num_kv_pages_per_block``, ``num_queries_per_block``, ``vmem_limit_bytes``)
are validated like upstream and otherwise ignored: the HIP schedule balances
work itself.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib, tuned

DEFAULT_MASK_VALUE = -0.7 * float(torch.finfo(torch.float32).max)  # ragged_paged_attention.py:32

_KV_DTYPES = {torch.bfloat16: _lib.RPA_KV_BF16, torch.float8_e4m3fn: _lib.RPA_KV_FP8_E4M3,
              torch.uint8: _lib.RPA_KV_FP8_E4M3}

_workspaces: dict[tuple[int, int], torch.Tensor] = {}
_ws_need: dict[int, int] = {}  # device index -> workspace bytes (depends only on the device)


def _require_cuda(name: str, t: torch.Tensor) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a GPU device, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def static_validate_inputs(q, kv_pages, kv_lens, page_indices, cu_q_lens, num_seqs, *,
                           sm_scale=None, sliding_window=None, soft_cap=None, mask_value=None,
                           k_scale=None, v_scale=None, num_kv_pages_per_block=None,
                           num_queries_per_block=None, vmem_limit_bytes=None) -> None:
    """Shape/dtype checks of ``static_validate_inputs`` (ragged_paged_attention.py:216-287)."""
    _, num_q_heads, head_dim = q.shape
    _, _, num_combined_kv_heads, head_dim_k = kv_pages.shape
    if num_combined_kv_heads % 2:
        raise ValueError(f"num_combined_kv_heads={num_combined_kv_heads} must be even")
    if not (isinstance(k_scale, float) or k_scale is None):
        raise ValueError(f"k_scale={k_scale!r} must be a float or None")
    if not (isinstance(v_scale, float) or v_scale is None):
        raise ValueError(f"v_scale={v_scale!r} must be a float or None")
    num_kv_heads = num_combined_kv_heads // 2
    max_num_seqs, pages_per_seq = page_indices.shape
    if tuple(num_seqs.shape) != (1,):
        raise ValueError(f"num_seqs.shape={tuple(num_seqs.shape)} must be (1,)")
    if head_dim_k != head_dim:
        raise ValueError(f"Q head_dim {head_dim} must be the same as that of K/V {head_dim_k}.")
    if tuple(kv_lens.shape) != (max_num_seqs,):
        raise ValueError(
            f"Expected kv_lens.shape={tuple(kv_lens.shape)} to be ({max_num_seqs},) where"
            " `max_num_seqs` is `page_indices.shape[0]`.")
    if tuple(cu_q_lens.shape) != (max_num_seqs + 1,):
        raise ValueError(
            f"Expected cu_q_lens.shape={tuple(cu_q_lens.shape)} to be ({max_num_seqs + 1},)  where"
            " `max_num_seqs` is `page_indices.shape[0]`.")
    if kv_lens.dtype != torch.int32 or page_indices.dtype != torch.int32 or cu_q_lens.dtype != torch.int32:
        raise ValueError(
            "The dtype of `kv_lens`, `page_indices`, and `cu_q_lens` must be"
            f" int32. Got kv_lens.dtype={kv_lens.dtype}, page_indices.dtype={page_indices.dtype},"
            f" cu_q_lens.dtype={cu_q_lens.dtype}.")
    if num_q_heads % num_kv_heads != 0:
        raise ValueError(f"num_q_heads={num_q_heads} must be divisible by num_kv_heads={num_kv_heads}")
    if sliding_window is not None and sliding_window <= 0:
        raise ValueError(f"sliding_window={sliding_window} must be positive.")
    if soft_cap is not None and soft_cap == 0.0:
        raise ValueError(f"soft_cap={soft_cap} must not be 0.0.")
    if num_kv_pages_per_block is not None and not 0 < num_kv_pages_per_block <= pages_per_seq:
        raise ValueError(f"num_kv_pages_per_block={num_kv_pages_per_block} must be in range (0, {pages_per_seq}].")
    if num_queries_per_block is not None and num_queries_per_block <= 0:
        raise ValueError(f"num_queries_per_block={num_queries_per_block} must be positive.")
    if vmem_limit_bytes is not None and vmem_limit_bytes <= 0:
        raise ValueError(f"vmem_limit_bytes={vmem_limit_bytes} must be positive.")


def dynamic_validate_inputs(q, kv_pages, kv_lens, page_indices, cu_q_lens, num_seqs, **kwargs) -> None:
    """``dynamic_validate_inputs`` (ragged_paged_attention.py:152-212); reads metadata to the host."""
    static_validate_inputs(q, kv_pages, kv_lens, page_indices, cu_q_lens, num_seqs, **kwargs)
    max_num_batched_tokens = q.shape[0]
    page_size = kv_pages.shape[1]
    max_num_seqs, pages_per_seq = page_indices.shape
    n = int(num_seqs.reshape(-1)[0].item())
    if n > max_num_seqs:
        raise ValueError(f"num_seqs[0]={n} must be less or equal to max_num_seqs={max_num_seqs}")
    lens = kv_lens.cpu()
    cu = cu_q_lens.cpu()
    max_kv_len = int(lens.max().item()) if lens.numel() else 0
    min_pages_per_seq = -(-max_kv_len // page_size)
    if pages_per_seq < min_pages_per_seq:
        raise ValueError(
            f"pages_per_seq={pages_per_seq} must be greater or equal to"
            f" min_pages_per_seq={min_pages_per_seq} given max_kv_len={max_kv_len} and page_size={page_size}.")
    if int(cu[n]) > max_num_batched_tokens:
        raise ValueError(f"Total q tokens {int(cu[n])} must be less or equal to"
                         f" max_num_batched_tokens={max_num_batched_tokens}.")
    for i in range(n):
        q_len = int(cu[i + 1]) - int(cu[i])
        kv_len = int(lens[i])
        if q_len > kv_len:
            raise ValueError(f"q_len={q_len} must be less or equal to kv_len={kv_len} at sequence {i}.")


def make_shape(q, kv_pages, page_indices) -> _lib.RpaShape:
    T, Hq, D = q.shape
    P, S, C, _ = kv_pages.shape
    n_max, pps = page_indices.shape
    kvd = _KV_DTYPES.get(kv_pages.dtype)
    if kvd is None:
        raise ValueError(f"kv_pages dtype {kv_pages.dtype} is not bf16 or fp8-e4m3")
    return _lib.RpaShape(T, Hq, C // 2, D, P, S, n_max, pps, kvd)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_get_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device


def _current_stream(dev: int) -> int:
    """The current stream's raw handle on device ``dev`` (torch's internal accessor when present:
    no Stream object per call)."""
    if _raw_stream is not None:
        return _raw_stream(dev)
    return torch.cuda.current_stream(dev).cuda_stream


_ws_fast: dict[tuple[int, int], tuple[int, int]] = {}


def _workspace_ptr(shape: _lib.RpaShape, dev: int, stream: int) -> tuple[int, int]:
    """(pointer, bytes) of the cached workspace of (device, stream)."""
    hit = _ws_fast.get((dev, stream))
    if hit is None:
        ws = workspace_for(shape, torch.device("cuda", dev), stream)
        hit = _ws_fast[(dev, stream)] = (ws.data_ptr(), ws.numel())
    return hit


_fns: tuple | None = None


def _entry_points() -> tuple:
    """(rpa_ragged_paged_attention, rpa_ragged_paged_attention_timed) of the loaded library."""
    global _fns
    if _fns is None:
        lib = _lib.load()
        _fns = (lib.rpa_ragged_paged_attention, lib.rpa_ragged_paged_attention_timed)
    return _fns


def workspace_for(shape: _lib.RpaShape, device: torch.device, stream: int) -> torch.Tensor:
    """Cached per-(device, stream) workspace; calls that share one must not overlap.  Its size
    depends only on the device (the persistent grid), so it is asked for once per device."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    ws = _workspaces.get((index, stream))
    if ws is not None and ws.numel() >= _ws_need[index]:
        return ws
    lib = _lib.load()
    need = lib.rpa_workspace_size(ctypes.byref(shape))
    if need == 0:
        _lib.check(-1)
    _ws_need[index] = need
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=device)
        _lib.check(lib.rpa_workspace_init(ws.data_ptr(), ws.numel(), stream))
        _workspaces[(index, stream)] = ws
        _ws_fast.pop((index, stream), None)
    return ws


def _static_plan(q, kv_pages, kv_lens, page_indices, cu_q_lens, num_seqs, kv_scales, knobs: dict) -> tuple:
    """Validate everything that depends only on shapes, dtypes, devices and the scalar knobs (the
    reference's static checks, :216-287, plus this build's), and build the ctypes structs.
    Returns (shape, options)."""
    static_validate_inputs(q, kv_pages, kv_lens, page_indices, cu_q_lens, num_seqs, **{
        k: knobs[k] for k in ("sm_scale", "sliding_window", "soft_cap", "mask_value", "k_scale", "v_scale",
                              "num_kv_pages_per_block", "num_queries_per_block", "vmem_limit_bytes")})
    for name, t in (("q", q), ("kv_pages", kv_pages), ("kv_lens", kv_lens), ("page_indices", page_indices),
                    ("cu_q_lens", cu_q_lens), ("num_seqs", num_seqs)):
        _require_cuda(name, t)
        if t.device != q.device:
            raise ValueError(f"{name} is on {t.device}, q on {q.device}")
    if q.dtype != torch.bfloat16:
        raise ValueError(f"q dtype {q.dtype} must be bfloat16")
    if num_seqs.dtype != torch.int32:
        raise ValueError(f"num_seqs dtype {num_seqs.dtype} must be int32")
    shape = make_shape(q, kv_pages, page_indices)
    if kv_scales is not None:
        if shape.kv_dtype != _lib.RPA_KV_FP8_E4M3:
            raise ValueError("kv_scales requires fp8 kv_pages")
        _require_cuda("kv_scales", kv_scales)
        if kv_scales.dtype != torch.float32 or tuple(kv_scales.shape) != (shape.total_pages, shape.num_kv_heads, 2):
            raise ValueError(f"kv_scales must be float32 [{shape.total_pages}, {shape.num_kv_heads}, 2]")
        if knobs["k_scale"] is not None or knobs["v_scale"] is not None:
            raise ValueError("pass either per-page kv_scales or scalar k_scale/v_scale, not both")
    # tuning knobs: the caller's, else the tuned table's entry for this shape, else the defaults
    tuned_knobs = tuned.get_tuned_knobs("fp8" if shape.kv_dtype == _lib.RPA_KV_FP8_E4M3 else "bf16",
                                        shape.num_q_heads // shape.num_kv_heads, shape.page_size, shape.num_tokens)
    wpc = knobs["waves_per_cu"] if knobs["waves_per_cu"] is not None else tuned_knobs["waves_per_cu"]
    tiles = knobs["prefill_tiles"] if knobs["prefill_tiles"] is not None else tuned_knobs["prefill_tiles"]
    cost = knobs["prefill_cost"] if knobs["prefill_cost"] is not None else tuned_knobs["prefill_cost"]
    if not (isinstance(wpc, int) and 0 <= wpc <= 8):
        raise ValueError(f"waves_per_cu={wpc!r} must be an int in [0, 8]")
    # True / 0: the library's choice; 1: the prefill kernel; 2: the attention kernel's own prefill
    # tiles (two 4-wave workgroups per CU where they apply); 3: the attention kernel's tiles in one
    # 8-wave workgroup per CU; False / -1: causal row blocks of the stream-K role
    tiles = {True: 0, False: -1}.get(tiles, tiles) if isinstance(tiles, bool) else tiles
    if tiles not in (-1, 0, 1, 2, 3):
        raise ValueError(f"prefill_tiles={tiles!r} must be a bool or one of -1, 0, 1, 2, 3")
    if not (0.0 <= float(cost) <= 64.0):
        raise ValueError(f"prefill_cost={cost!r} must be in [0, 64]")
    mask_value = knobs["mask_value"]
    if mask_value is None:
        mask_value = DEFAULT_MASK_VALUE
    k_scale, v_scale = knobs["k_scale"], knobs["v_scale"]
    opts = _lib.RpaOptions(
        float(knobs["sm_scale"]), int(knobs["sliding_window"] or 0), float(knobs["soft_cap"] or 0.0),
        1, float(mask_value),
        int(k_scale is not None), float(k_scale if k_scale is not None else 1.0),
        int(v_scale is not None), float(v_scale if v_scale is not None else 1.0),
        int(wpc), int(tiles), float(cost),
    )
    return shape, opts


# Validated (shape, options) per call signature: shapes, dtypes, devices and knobs.  A serving loop
# calls with the same signature every step, so the checks and struct building above run once.
_plans: dict[tuple, tuple] = {}


def ragged_paged_attention(
    q: torch.Tensor,             # bf16 [max_num_batched_tokens, num_q_heads, head_dim]
    kv_pages: torch.Tensor,      # bf16 | float8_e4m3fn | uint8 (e4m3 codes) [pages, page_size, 2*Hkv, D]
    kv_lens: torch.Tensor,       # i32[max_num_seqs]
    page_indices: torch.Tensor,  # i32[max_num_seqs, pages_per_seq]
    cu_q_lens: torch.Tensor,     # i32[max_num_seqs + 1]
    num_seqs: torch.Tensor,      # i32[1]
    *,
    sm_scale: float = 1.0,
    sliding_window: int | None = None,
    soft_cap: float | None = None,
    mask_value: float | None = DEFAULT_MASK_VALUE,
    k_scale: float | None = None,
    v_scale: float | None = None,
    num_kv_pages_per_block: int | None = None,
    num_queries_per_block: int | None = None,
    vmem_limit_bytes: int | None = None,
    kv_scales: torch.Tensor | None = None,   # f32 [pages, Hkv, 2] per-(page, kv head) K/V scales
    out: torch.Tensor | None = None,
    kernel_events: tuple | None = None,      # (begin, end) events around the attention kernel: torch.cuda.Event
                                             # or timing.KernelEvent (anything with a .cuda_event handle)
    waves_per_cu: int | None = None,         # tuning knobs (rpa_options_t); None = the tuned table's entry
    prefill_tiles: bool | int | None = None, # 1 prefill kernel, 2/3 in-kernel tiles, True/0 auto, False/-1 rows
    prefill_cost: float | None = None,
) -> torch.Tensor:
    """Ragged paged attention (mixed prefill and decode) on MI355X.

    Semantics of ``ref_ragged_paged_attention`` (ragged_paged_attention.py:73-148).
    Returns a new ``[T, Hq, D]`` bf16 tensor (or fills ``out``); rows at or past
    ``cu_q_lens[num_seqs]`` are zero.  The Pallas block sizes are validated like upstream
    and have no effect; the schedule knobs ``waves_per_cu`` / ``prefill_tiles`` /
    ``prefill_cost`` take their place (``tpu_cake_amd.tuned`` holds per-shape values).
    """
    dev = q.get_device()  # -1 for a CPU tensor: rejected by the plan's checks
    sig = (q.shape, q.dtype, dev, kv_pages.shape, kv_pages.dtype, kv_pages.get_device(), kv_lens.shape,
           kv_lens.dtype, kv_lens.get_device(), page_indices.shape, page_indices.dtype, page_indices.get_device(),
           cu_q_lens.shape, cu_q_lens.dtype, cu_q_lens.get_device(), num_seqs.shape, num_seqs.dtype,
           num_seqs.get_device(),
           None if kv_scales is None else (kv_scales.shape, kv_scales.dtype, kv_scales.get_device()),
           sm_scale, sliding_window, soft_cap, mask_value, k_scale, v_scale, num_kv_pages_per_block,
           num_queries_per_block, vmem_limit_bytes, waves_per_cu, prefill_tiles, prefill_cost)
    plan = _plans.get(sig)
    if plan is None:
        plan = _static_plan(q, kv_pages, kv_lens, page_indices, cu_q_lens, num_seqs, kv_scales, dict(
            sm_scale=sm_scale, sliding_window=sliding_window, soft_cap=soft_cap, mask_value=mask_value,
            k_scale=k_scale, v_scale=v_scale, num_kv_pages_per_block=num_kv_pages_per_block,
            num_queries_per_block=num_queries_per_block, vmem_limit_bytes=vmem_limit_bytes,
            waves_per_cu=waves_per_cu, prefill_tiles=prefill_tiles, prefill_cost=prefill_cost))
        if len(_plans) > 256:
            _plans.clear()
        _plans[sig] = plan
    shape, opts = plan
    # per call: what the signature does not fix
    if not (q.is_contiguous() and kv_pages.is_contiguous() and kv_lens.is_contiguous()
            and page_indices.is_contiguous() and cu_q_lens.is_contiguous() and num_seqs.is_contiguous()
            and (kv_scales is None or kv_scales.is_contiguous())):
        for name, t in (("q", q), ("kv_pages", kv_pages), ("kv_lens", kv_lens), ("page_indices", page_indices),
                        ("cu_q_lens", cu_q_lens), ("num_seqs", num_seqs), ("kv_scales", kv_scales)):
            if t is not None:
                _require_cuda(name, t)
    if out is None:
        out = torch.empty_like(q)
    elif (out.shape != q.shape or out.dtype != q.dtype or out.get_device() != dev or not out.is_contiguous()
          or out.data_ptr() == q.data_ptr()):
        raise ValueError("out must be a separate contiguous tensor shaped like q on q's device")
    if dev != _get_device():
        with torch.cuda.device(dev):
            return ragged_paged_attention(q, kv_pages, kv_lens, page_indices, cu_q_lens, num_seqs, sm_scale=sm_scale,
                                          sliding_window=sliding_window, soft_cap=soft_cap, mask_value=mask_value,
                                          k_scale=k_scale, v_scale=v_scale,
                                          num_kv_pages_per_block=num_kv_pages_per_block,
                                          num_queries_per_block=num_queries_per_block,
                                          vmem_limit_bytes=vmem_limit_bytes, kv_scales=kv_scales, out=out,
                                          kernel_events=kernel_events, waves_per_cu=waves_per_cu,
                                          prefill_tiles=prefill_tiles, prefill_cost=prefill_cost)
    stream = _current_stream(dev)
    ws_ptr, ws_bytes = _workspace_ptr(shape, dev, stream)
    fn = _entry_points()
    args = (shape, opts, q.data_ptr(), kv_pages.data_ptr(),
            kv_scales.data_ptr() if kv_scales is not None else None,
            kv_lens.data_ptr(), page_indices.data_ptr(), cu_q_lens.data_ptr(), num_seqs.data_ptr(),
            out.data_ptr(), ws_ptr, ws_bytes, stream)
    if kernel_events is None:
        rc = fn[0](*args)
    else:
        begin, end = kernel_events
        if not begin.cuda_event or not end.cuda_event:
            raise ValueError("kernel_events must be recorded once before use (HIP events are created lazily)")
        rc = fn[1](*args, begin.cuda_event, end.cuda_event)
    if rc:
        _lib.check(rc)
    return out


class CapturedCalls:
    """Several ``ragged_paged_attention`` calls captured into one HIP graph over fixed buffers.

    The form a serving loop uses when its whole step is a graph: one call per layer, each over its
    own queries, K/V pool and output, usually sharing the step's metadata tensors.  The loop writes
    each step's values and metadata into the same tensors and calls ``replay()``; the graph re-runs
    every call's kernels on what those tensors hold, for one graph launch.  Capture happens on a
    stream of this object (default priority) after one warm-up run of every call on it, so the
    validated plans and the stream's workspace (allocated and initialised by
    ``rpa_workspace_init``) exist beforehand: the graph records only the calls' kernel launches --
    no allocation, no memset node.  The calls run in list order on the one stream and share its
    workspace, so replays must not overlap other calls on it.  Metadata changes keep the shapes
    (``num_seqs``, ``kv_lens``, ``cu_q_lens`` and ``page_indices`` values may change; their sizes,
    the dtypes and the knobs are fixed at capture).

    ``calls`` is a sequence of ``(args, kwargs)`` pairs, ``args`` the operator's six positionals;
    a call without ``out`` in its keywords gets a new output tensor.  ``outs`` holds the outputs.
    """

    def __init__(self, calls):
        calls = list(calls)
        if not calls:
            raise ValueError("no calls to capture")
        self._calls = []
        for args, kwargs in calls:
            if len(args) != 6:
                raise ValueError("each call takes the operator's six positional arguments")
            if kwargs.get("kernel_events") is not None:
                raise ValueError("a captured call takes no kernel_events")
            out = kwargs.get("out")
            if out is None:
                out = torch.empty_like(args[0])
            self._calls.append((tuple(args), dict(kwargs, out=out)))
        self.outs = [kw["out"] for _, kw in self._calls]
        dev = self._calls[0][0][0].device
        self.stream = torch.cuda.Stream(device=dev)
        self.stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(self.stream):
            for args, kwargs in self._calls:  # plans + this stream's workspace
                ragged_paged_attention(*args, **kwargs)
        self.stream.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            for args, kwargs in self._calls:
                ragged_paged_attention(*args, **kwargs)

    def replay(self) -> list:
        """Launch the captured calls (ordered after the current stream's work); returns ``outs``."""
        self.graph.replay()
        return self.outs


class CapturedCall(CapturedCalls):
    """One ``ragged_paged_attention`` call captured into a HIP graph over fixed buffers
    (``CapturedCalls`` with one call; ``replay()`` returns ``out``).

    A graph launch costs more host time on this platform than the operator's own eager call, and
    each replay adds a few microseconds of device time, so a graph of one call is slower than the
    eager call it captures (small calls are host-bound at the graph-launch rate); a graph holding a
    whole step's calls (``CapturedCalls``) pays that launch once for all of them.
    """

    def __init__(self, q, kv_pages, kv_lens, page_indices, cu_q_lens, num_seqs, *, out=None, **kwargs):
        super().__init__([((q, kv_pages, kv_lens, page_indices, cu_q_lens, num_seqs), dict(kwargs, out=out))])
        self.out = self.outs[0]

    def replay(self) -> torch.Tensor:
        """Launch the captured call (ordered after the current stream's work) and return ``out``."""
        self.graph.replay()
        return self.out


class PreparedCall:
    """One ``ragged_paged_attention`` call with its host work done once, for a serving loop that
    passes the same tensors every step.

    Construction runs the call once through the operator (every check, the plan, the current
    stream's workspace) and keeps the library entry point, the shape and option structures, each
    tensor's address, the workspace and the stream as ready foreign-call arguments; ``__call__``
    launches the kernels with one foreign call.  Fixed at construction: the tensors (their storage,
    shapes and dtypes), the keywords and the stream (the current one then); free between calls:
    every value they hold -- queries, K/V pages and all metadata.  Calls on one stream share its
    workspace and must not overlap.  Unlike ``CapturedCall`` no graph is involved: the launches are
    ordinary stream work, so the call costs less host time than a graph replay on this platform.
    """

    def __init__(self, q, kv_pages, kv_lens, page_indices, cu_q_lens, num_seqs, *, out=None, kv_scales=None,
                 **kwargs):
        if kwargs.get("kernel_events") is not None:
            raise ValueError("a prepared call takes no kernel_events")
        self.out = out if out is not None else torch.empty_like(q)
        ragged_paged_attention(q, kv_pages, kv_lens, page_indices, cu_q_lens, num_seqs, out=self.out,
                               kv_scales=kv_scales, **kwargs)
        knobs = dict(sm_scale=1.0, sliding_window=None, soft_cap=None, mask_value=DEFAULT_MASK_VALUE, k_scale=None,
                     v_scale=None, num_kv_pages_per_block=None, num_queries_per_block=None, vmem_limit_bytes=None,
                     waves_per_cu=None, prefill_tiles=None, prefill_cost=None)
        unknown = set(kwargs) - set(knobs)
        if unknown:
            raise TypeError(f"unexpected keyword arguments {sorted(unknown)}")
        knobs.update(kwargs)
        self._shape, self._opts = _static_plan(q, kv_pages, kv_lens, page_indices, cu_q_lens, num_seqs, kv_scales,
                                               knobs)
        dev = q.get_device()
        self.stream = _current_stream(dev)
        ws_ptr, ws_bytes = _workspace_ptr(self._shape, dev, self.stream)
        # a function object of its own without argument types: the prepared ctypes values pass as-is
        fn = _lib.load()["rpa_ragged_paged_attention"]
        fn.restype = ctypes.c_int
        vp = ctypes.c_void_p
        self._fn = fn
        self._keep = (q, kv_pages, kv_lens, page_indices, cu_q_lens, num_seqs, kv_scales, self.out)
        self._args = (ctypes.byref(self._shape), ctypes.byref(self._opts), vp(q.data_ptr()), vp(kv_pages.data_ptr()),
                      vp(kv_scales.data_ptr() if kv_scales is not None else None), vp(kv_lens.data_ptr()),
                      vp(page_indices.data_ptr()), vp(cu_q_lens.data_ptr()), vp(num_seqs.data_ptr()),
                      vp(self.out.data_ptr()), vp(ws_ptr), ctypes.c_size_t(ws_bytes), vp(self.stream))

    def __call__(self) -> torch.Tensor:
        """Launch the call on its stream and return ``out``."""
        rc = self._fn(*self._args)
        if rc:
            _lib.check(rc)
        return self.out


def read_error_word(device: torch.device | None = None) -> int:
    """Synchronously read the device-side metadata error word of the current stream's workspace."""
    device = device or torch.device("cuda", torch.cuda.current_device())
    stream = torch.cuda.current_stream(device).cuda_stream
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _workspaces.get(key)
    if ws is None:
        return 0
    word = ctypes.c_int32(0)
    _lib.check(_lib.load().rpa_read_error_word(ws.data_ptr(), ws.numel(), ctypes.byref(word), stream))
    return int(word.value)


def gather_kv(kv_pages, kv_lens, page_indices, num_seqs) -> torch.Tensor:
    """Dense ``[sum(kv_lens[:num_seqs]), 2*Hkv, D]`` copy of the K/V rows the kernel reads."""
    for name, t in (("kv_pages", kv_pages), ("kv_lens", kv_lens), ("page_indices", page_indices),
                    ("num_seqs", num_seqs)):
        _require_cuda(name, t)
    n = int(num_seqs.reshape(-1)[0].item())
    rows = int(kv_lens[:n].to(torch.int64).sum().item())
    P, S, C, D = kv_pages.shape
    dense = torch.zeros((rows, C, D), dtype=kv_pages.dtype, device=kv_pages.device)
    dummy_q = torch.empty((0, C // 2, D), dtype=torch.bfloat16, device=kv_pages.device)
    shape = make_shape(dummy_q, kv_pages, page_indices)
    with torch.cuda.device(kv_pages.device):
        stream = torch.cuda.current_stream(kv_pages.device).cuda_stream
        ws = workspace_for(shape, kv_pages.device, stream)
        _lib.check(_lib.load().rpa_gather_kv(
            ctypes.byref(shape), kv_pages.data_ptr(), kv_lens.data_ptr(), page_indices.data_ptr(),
            num_seqs.data_ptr(), dense.data_ptr() if rows else None, rows, ws.data_ptr(), ws.numel(), stream))
    return dense


def case_to_device(case, device="cuda") -> dict:
    """Host ``RpaCase`` (tpu_cake_amd.workloads) -> dict of device tensors for the operator."""
    import numpy as np

    dev = torch.device(device)
    q = torch.from_numpy(np.ascontiguousarray(case.q).view(np.int16)).view(torch.bfloat16).to(dev)
    if case.kv_dtype == "fp8":
        kv = torch.from_numpy(np.ascontiguousarray(case.kv_pages)).view(torch.float8_e4m3fn).to(dev)
    else:
        kv = torch.from_numpy(np.ascontiguousarray(case.kv_pages).view(np.int16)).view(torch.bfloat16).to(dev)
    d = {
        "q": q,
        "kv_pages": kv,
        "kv_lens": torch.from_numpy(np.ascontiguousarray(case.kv_lens, dtype=np.int32)).to(dev),
        "page_indices": torch.from_numpy(np.ascontiguousarray(case.page_indices, dtype=np.int32)).to(dev),
        "cu_q_lens": torch.from_numpy(np.ascontiguousarray(case.cu_q_lens, dtype=np.int32)).to(dev),
        "num_seqs": torch.from_numpy(np.ascontiguousarray(case.num_seqs, dtype=np.int32)).to(dev),
    }
    if case.kv_scales is not None:
        d["kv_scales"] = torch.from_numpy(np.ascontiguousarray(case.kv_scales, dtype=np.float32)).to(dev)
    return d


def run_case(case, device="cuda", **kwargs) -> torch.Tensor:
    """Run the operator on a host ``RpaCase``; returns the device output."""
    d = case_to_device(case, device)
    kv_scales = d.pop("kv_scales", None)
    return ragged_paged_attention(d["q"], d["kv_pages"], d["kv_lens"], d["page_indices"], d["cu_q_lens"],
                                  d["num_seqs"], sm_scale=case.sm_scale, kv_scales=kv_scales, **kwargs)


def attention_grid(case, knobs: dict | None = None, cus: int = 0) -> tuple[int, int]:
    """(workgroups, waves per workgroup) of the attention launch the library makes for a host
    ``RpaCase`` with the schedule knobs ``knobs`` (``waves_per_cu`` / ``prefill_tiles`` /
    ``prefill_cost``), on a device of ``cus`` compute units at the kernel's nominal occupancy, or
    on the current GPU when ``cus`` is 0 (``rpa_attention_grid``)."""
    k = tuned.validate_entry(dict(knobs or {}))
    T, Hq, D = case.q.shape
    P, S, C, _ = case.kv_pages.shape
    n_max, pps = case.page_indices.shape
    shape = _lib.RpaShape(T, Hq, C // 2, D, P, S, n_max, pps,
                          _lib.RPA_KV_FP8_E4M3 if case.kv_dtype == "fp8" else _lib.RPA_KV_BF16)
    opts = _lib.RpaOptions(sm_scale=float(case.sm_scale), waves_per_cu=int(k["waves_per_cu"]),
                           prefill_tiles=int(k["prefill_tiles"]), prefill_cost=float(k["prefill_cost"]))
    grid, waves = ctypes.c_int32(0), ctypes.c_int32(0)
    lib = _lib.load()
    _lib.check(lib.rpa_attention_grid(ctypes.byref(shape), ctypes.byref(opts), int(cus), ctypes.byref(grid),
                                      ctypes.byref(waves)))
    return grid.value, waves.value


def default_sm_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)

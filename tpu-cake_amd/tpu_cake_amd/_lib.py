"""ctypes binding of ``librpa.so`` (the C ABI declared in ``include/rpa.h``).

The library is built in-tree next to this file (``tpu_cake_amd/librpa.so``,
see ``tpu_cake_amd.build``); ``RPA_LIB`` overrides the path.  There is no
fallback: if the library is missing every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
import threading

LIB_PATH = pathlib.Path(__file__).with_name("librpa.so")
ABI_VERSION = 2

RPA_OK = 0
RPA_KV_BF16 = 0
RPA_KV_FP8_E4M3 = 1

# Every symbol include/rpa.h declares.
EXPORTED_SYMBOLS = (
    "rpa_abi_version",
    "rpa_last_error",
    "rpa_workspace_size",
    "rpa_workspace_init",
    "rpa_ragged_paged_attention",
    "rpa_ragged_paged_attention_timed",
    "rpa_ragged_paged_attention_noalloc",
    "rpa_gather_kv",
    "rpa_read_error_word",
    "rpa_fused_workspace_size",
    "rpa_inkling_fused_decode",
    "rpa_inkling_workspace_size",
    "rpa_inkling_decode",
    "rpa_attention_grid",
    "rpa_timeline_read",
)


class RpaShape(ctypes.Structure):
    _fields_ = [
        ("num_tokens", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("total_pages", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("max_num_seqs", ctypes.c_int32),
        ("pages_per_seq", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
    ]


class RpaOptions(ctypes.Structure):
    _fields_ = [
        ("sm_scale", ctypes.c_float),
        ("sliding_window", ctypes.c_int32),
        ("soft_cap", ctypes.c_float),
        ("has_mask_value", ctypes.c_int32),
        ("mask_value", ctypes.c_float),
        ("has_k_scale", ctypes.c_int32),
        ("k_scale", ctypes.c_float),
        ("has_v_scale", ctypes.c_int32),
        ("v_scale", ctypes.c_float),
        # tuning knobs (ABI 2; 0 = library default)
        ("waves_per_cu", ctypes.c_int32),
        ("prefill_tiles", ctypes.c_int32),
        ("prefill_cost", ctypes.c_float),
    ]


class RpaFusedShape(ctypes.Structure):
    _fields_ = [
        ("num_seqs", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("total_pages", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("cache_width", ctypes.c_int32),
        ("page_entries", ctypes.c_int32),
        ("pages_per_seq", ctypes.c_int32),
        ("relative_dim", ctypes.c_int32),
        ("relative_extent", ctypes.c_int32),
    ]


class RpaInklingShape(ctypes.Structure):
    """include/rpa.h: rpa_inkling_shape_t (the v1 Inkling decode contract)."""

    _fields_ = [
        ("num_seqs", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("total_pages", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("pages_per_seq", ctypes.c_int32),
        ("bias_len", ctypes.c_int32),
    ]


class RpaError(RuntimeError):
    """A nonzero return from librpa (message from ``rpa_last_error``)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"librpa error {code}: {message}")
        self.code = code


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path() -> pathlib.Path:
    return pathlib.Path(os.environ.get("RPA_LIB", str(LIB_PATH)))


def load() -> ctypes.CDLL:
    """Load ``librpa.so`` once; raise if it is missing or has the wrong ABI."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            raise RuntimeError(
                f"librpa.so not found at {path}; build it with `python -m tpu_cake_amd.build` "
                "(there is no CPU fallback)"
            )
        lib = ctypes.CDLL(str(path))
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        i32p = ctypes.POINTER(ctypes.c_int32)
        lib.rpa_abi_version.restype = ctypes.c_int
        lib.rpa_abi_version.argtypes = []
        lib.rpa_last_error.restype = ctypes.c_char_p
        lib.rpa_last_error.argtypes = []
        lib.rpa_workspace_size.restype = sz
        lib.rpa_workspace_size.argtypes = [ctypes.POINTER(RpaShape)]
        lib.rpa_workspace_init.restype = ctypes.c_int
        lib.rpa_workspace_init.argtypes = [vp, sz, vp]
        lib.rpa_ragged_paged_attention.restype = ctypes.c_int
        lib.rpa_ragged_paged_attention.argtypes = [
            ctypes.POINTER(RpaShape), ctypes.POINTER(RpaOptions), vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp,
        ]
        lib.rpa_ragged_paged_attention_timed.restype = ctypes.c_int
        lib.rpa_ragged_paged_attention_timed.argtypes = [
            ctypes.POINTER(RpaShape), ctypes.POINTER(RpaOptions), vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp, vp, vp,
        ]
        lib.rpa_ragged_paged_attention_noalloc.restype = ctypes.c_int
        lib.rpa_ragged_paged_attention_noalloc.argtypes = [
            ctypes.POINTER(RpaShape), ctypes.POINTER(RpaOptions), vp, vp, vp, vp, vp, vp, vp, vp, vp,
        ]
        lib.rpa_gather_kv.restype = ctypes.c_int
        lib.rpa_gather_kv.argtypes = [ctypes.POINTER(RpaShape), vp, vp, vp, vp, vp, ctypes.c_int64, vp, sz, vp]
        lib.rpa_read_error_word.restype = ctypes.c_int
        lib.rpa_read_error_word.argtypes = [vp, sz, i32p, vp]
        lib.rpa_fused_workspace_size.restype = sz
        lib.rpa_fused_workspace_size.argtypes = [ctypes.POINTER(RpaFusedShape)]
        lib.rpa_inkling_fused_decode.restype = ctypes.c_int
        # shape, sm_scale, 12 tensors (queries .. out), workspace, workspace_bytes, stream
        lib.rpa_inkling_fused_decode.argtypes = [ctypes.POINTER(RpaFusedShape), ctypes.c_float] + [vp] * 13 + [sz, vp]
        lib.rpa_inkling_workspace_size.restype = sz
        lib.rpa_inkling_workspace_size.argtypes = [ctypes.POINTER(RpaInklingShape)]
        lib.rpa_attention_grid.restype = ctypes.c_int
        lib.rpa_attention_grid.argtypes = [ctypes.POINTER(RpaShape), ctypes.POINTER(RpaOptions), ctypes.c_int32,
                                           i32p, i32p]
        lib.rpa_timeline_read.restype = ctypes.c_int
        lib.rpa_timeline_read.argtypes = [ctypes.POINTER(ctypes.c_int64), ctypes.c_int32, vp]
        lib.rpa_inkling_decode.restype = ctypes.c_int
        lib.rpa_inkling_decode.argtypes = [ctypes.POINTER(RpaInklingShape), ctypes.c_float] + [vp] * 8 + [sz, vp]
        version = lib.rpa_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{path}: ABI version {version}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def check(rc: int) -> None:
    if rc != RPA_OK:
        msg = load().rpa_last_error().decode(errors="replace")
        raise RpaError(rc, msg)

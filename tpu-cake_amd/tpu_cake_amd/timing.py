"""Timing-only HIP events for the kernel measurement hook.

``rpa_ragged_paged_attention_timed`` records two caller-owned events around the
attention kernel.  A default HIP event performs a system-scope release when it is
recorded (cache writeback and invalidate), which slows the work around it; events
created with ``hipEventDisableSystemFence`` record only the timestamp, so timing
every call of a benchmark does not change what is timed.  They are for timing
only: they do not make device memory visible to the host.
"""

from __future__ import annotations

import ctypes

HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000  # hip_runtime_api.h

_hip = None


def _runtime():
    """The HIP runtime already loaded by torch (soname libamdhip64.so.7)."""
    global _hip
    if _hip is None:
        import torch

        torch.cuda.init()
        lib = ctypes.CDLL("libamdhip64.so.7")
        lib.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
        lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        _hip = lib
    return _hip


class KernelEvent:
    """A HIP event on the current device for timing only (``.cuda_event`` is the handle)."""

    def __init__(self):
        hip = _runtime()
        handle = ctypes.c_void_p()
        rc = hip.hipEventCreateWithFlags(ctypes.byref(handle), HIP_EVENT_DISABLE_SYSTEM_FENCE)
        if rc != 0 or not handle.value:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
        self._hip = hip
        self.cuda_event = handle.value

    def record(self, stream=None) -> None:
        """Record on ``stream`` (a HIP stream handle; default: torch's current stream)."""
        if stream is None:
            import torch

            stream = torch.cuda.current_stream().cuda_stream
        rc = self._hip.hipEventRecord(self.cuda_event, stream)
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_time(self, end: "KernelEvent") -> float:
        """Milliseconds from this event to ``end`` (both recorded and complete)."""
        ms = ctypes.c_float()
        rc = self._hip.hipEventElapsedTime(ctypes.byref(ms), self.cuda_event, end.cuda_event)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return float(ms.value)

    def __del__(self):
        if getattr(self, "cuda_event", None):
            self._hip.hipEventDestroy(self.cuda_event)
            self.cuda_event = None

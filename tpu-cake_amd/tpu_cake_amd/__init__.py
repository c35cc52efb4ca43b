"""tpu_cake_amd: ragged paged attention (RPA) for AMD Instinct MI355X.

The hot path of sdrshn-nmbr/tpu-cake's Inkling RPA workload, rebuilt as
hand-written gfx950 HIP kernels (``librpa.so``, C ABI in ``include/rpa.h``)
behind the reference operator's Python surface (``tpu_cake_amd.ops``), and the
fused Inkling decode step (KV-cache write + relative-bias attention) behind the
reference's fused-plan surface (``tpu_cake_amd.fused``); the v1 Inkling decode
contract (``experiment inkling-rpa``) runs through ``tpu_cake_amd.inkling``.
"""

from . import fused, inkling  # noqa: F401

from .ops import (  # noqa: F401
    DEFAULT_MASK_VALUE,
    CapturedCall,
    CapturedCalls,
    PreparedCall,
    dynamic_validate_inputs,
    gather_kv,
    ragged_paged_attention,
    read_error_word,
    static_validate_inputs,
)

__all__ = [
    "CapturedCall",
    "CapturedCalls",
    "DEFAULT_MASK_VALUE",
    "PreparedCall",
    "fused",
    "inkling",
    "dynamic_validate_inputs",
    "gather_kv",
    "ragged_paged_attention",
    "read_error_word",
    "static_validate_inputs",
]

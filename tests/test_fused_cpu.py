"""The fused decode's host side on the CPU: the product preflight (tpu_cake_amd.fused) rejects the
reference's bad-metadata cases (tests/test_rpa_lowering.py:604-653) with its messages, and agrees
with the oracle's preflight on random corruptions of valid metadata."""

import numpy as np
import pytest

from oracle import rpa_fused_oracle as fo
from tpu_cake_amd import fused

from test_fused_oracle import _preflight_cases


def _args(inp):
    return [inp[k] for k in fused.INPUT_NAMES]


def test_product_preflight_matches_reference_cases():
    base, cases = _preflight_cases()
    fused.preflight(*_args(base))
    for inp, msg in cases:
        with pytest.raises(ValueError, match=msg):
            fused.preflight(*_args(inp))


def test_product_preflight_agrees_with_oracle_on_corruptions():
    rng = np.random.default_rng(7)
    base = fo.fused_inputs_like(1, nseq=5, hq=8, hkv=2, d=32, page_size=16, pool_pages=64,
                                lengths=[1, 16, 17, 40, 100], rel_dim=4, extent=32)
    for trial in range(200):
        inp = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in base.items()}
        field = ("page_indices", "kv_lengths", "cu_kv_lens")[trial % 3]
        arr = inp[field]
        i = int(rng.integers(0, arr.size))
        arr[i] = arr[i] + int(rng.integers(-3, 4)) if field != "page_indices" else int(rng.integers(-1, 66))
        def outcome(f):
            try:
                f(inp)
                return None
            except ValueError as e:
                return str(e)
        assert outcome(fo.preflight_fused_decode) == outcome(lambda x: fused.preflight(*_args(x))), (field, i)

"""The v1 Inkling wrapper's argument checks (tpu_cake_amd.inkling) raise the reference's
ValueErrors (src/tpu_cake/workloads/inkling_rpa.py:45-55) before touching the GPU."""

import pytest
import torch

from tpu_cake_amd import inkling


def _args(**kw):
    a = dict(query=torch.zeros(4, 4, 32), key_cache=torch.zeros(32, 16, 4, 32), value_cache=torch.zeros(32, 16, 4, 32),
             page_table=torch.zeros(4, 8, dtype=torch.int32), sequence_lengths=torch.ones(4, dtype=torch.int32),
             bias=torch.zeros(4, 128))
    a.update(kw)
    return a


@pytest.mark.parametrize("kw,msg", [
    (dict(value_cache=torch.zeros(32, 8, 4, 32)), "same page size"),
    (dict(key_cache=torch.zeros(32, 16, 4, 16), value_cache=torch.zeros(32, 16, 4, 16)), "head dimensions must match"),
    (dict(key_cache=torch.zeros(32, 16, 3, 32), value_cache=torch.zeros(32, 16, 3, 32)), "divide evenly"),
    (dict(bias=torch.zeros(3, 128)), "one row per query head"),
    (dict(value_cache=torch.zeros(32, 16, 2, 32)), "same shape on this backend"),
    (dict(), "contiguous CUDA"),
])
def test_reference_checks(kw, msg):
    with pytest.raises(ValueError, match=msg):
        inkling._check(**_args(**kw))

"""The C ABI: librpa.so loads, exports every entry point include/rpa.h declares, the ctypes
structs match the C layout, host-side argument checks fail before any GPU work, and the
work-decomposition math the kernels share passes the host checker.  No GPU needed."""

import ctypes
import pathlib
import re
import subprocess

import pytest

from tpu_cake_amd import _lib

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "rpa.h"


@pytest.fixture(scope="module")
def lib():
    if not _lib.library_path().exists():
        from tpu_cake_amd import build
        build.build()
    return _lib.load()


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(rpa_[a-z_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.library_path())], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (rpa_\w+)", out))
    missing = [s for s in declared_functions() if s not in exported]
    assert not missing, missing
    for s in declared_functions():
        assert hasattr(lib, s)


def test_abi_version(lib):
    assert lib.rpa_abi_version() == _lib.ABI_VERSION == 2


def test_struct_layout_matches_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "rpa.h"\n'
        "int main(void){\n"
        '  printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\\n", sizeof(rpa_shape_t),\n'
        "         offsetof(rpa_shape_t, kv_dtype),\n"
        "         sizeof(rpa_options_t), offsetof(rpa_options_t, mask_value), offsetof(rpa_options_t, v_scale),\n"
        "         offsetof(rpa_options_t, has_k_scale), offsetof(rpa_options_t, waves_per_cu),\n"
        "         offsetof(rpa_options_t, prefill_tiles), offsetof(rpa_options_t, prefill_cost),\n"
        "         sizeof(rpa_fused_shape_t),\n"
        "         offsetof(rpa_fused_shape_t, relative_extent), sizeof(rpa_inkling_shape_t),\n"
        "         offsetof(rpa_inkling_shape_t, bias_len));\n  return 0; }\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [ctypes.sizeof(_lib.RpaShape), _lib.RpaShape.kv_dtype.offset, ctypes.sizeof(_lib.RpaOptions),
            _lib.RpaOptions.mask_value.offset, _lib.RpaOptions.v_scale.offset, _lib.RpaOptions.has_k_scale.offset,
            _lib.RpaOptions.waves_per_cu.offset, _lib.RpaOptions.prefill_tiles.offset,
            _lib.RpaOptions.prefill_cost.offset, ctypes.sizeof(_lib.RpaFusedShape), _lib.RpaFusedShape.relative_extent.offset,
            ctypes.sizeof(_lib.RpaInklingShape), _lib.RpaInklingShape.bias_len.offset]
    assert got == want


def _shape(**kw):
    base = dict(num_tokens=4, num_q_heads=8, num_kv_heads=2, head_dim=128, total_pages=10, page_size=16,
                max_num_seqs=4, pages_per_seq=4, kv_dtype=0)
    base.update(kw)
    return _lib.RpaShape(**base)


@pytest.mark.parametrize("head_dim,kv_dtype", [(512, 0), (192, 0), (24, 0), (36, 0), (48, 1), (72, 1)])
def test_unsupported_head_dim_rejected_before_launch(lib, head_dim, kv_dtype):
    # built: 128, 256, and narrower multiples of 8 in [32, 128] (fp8: multiples of 16 in [64, 128])
    opts = _lib.RpaOptions(sm_scale=1.0)
    rc = lib.rpa_ragged_paged_attention(ctypes.byref(_shape(head_dim=head_dim, kv_dtype=kv_dtype)),
                                        ctypes.byref(opts), *([None] * 9), 0, None)
    assert rc == -2
    assert f"head_dim {head_dim}".encode() in lib.rpa_last_error()


@pytest.mark.parametrize("head_dim,kv_dtype", [(32, 0), (64, 0), (96, 0), (120, 0), (64, 1), (112, 1), (256, 0),
                                               (256, 1)])
def test_narrow_head_dims_pass_the_shape_check(lib, head_dim, kv_dtype):
    # the shape check accepts them: the call then stops at the missing workspace, before any launch
    opts = _lib.RpaOptions(sm_scale=1.0)
    rc = lib.rpa_ragged_paged_attention(ctypes.byref(_shape(head_dim=head_dim, kv_dtype=kv_dtype)),
                                        ctypes.byref(opts), *([None] * 9), 0, None)
    assert rc != -2, lib.rpa_last_error()


@pytest.mark.parametrize("bad,msg", [(dict(num_q_heads=6, num_kv_heads=4), b"divisible"),
                                     (dict(kv_dtype=7), b"kv_dtype"),
                                     (dict(page_size=0), b"non-positive")])
def test_invalid_shapes_rejected(lib, bad, msg):
    opts = _lib.RpaOptions(sm_scale=1.0)
    rc = lib.rpa_ragged_paged_attention(ctypes.byref(_shape(**bad)), ctypes.byref(opts), *([None] * 9), 0, None)
    assert rc == -1 and msg in lib.rpa_last_error()


@pytest.mark.parametrize("knob,msg", [(dict(waves_per_cu=9), b"waves_per_cu"), (dict(waves_per_cu=-1), b"waves_per_cu"),
                                      (dict(prefill_tiles=4), b"prefill_tiles"),
                                      (dict(prefill_cost=-0.5), b"prefill_cost")])
def test_invalid_tuning_knobs_rejected(lib, knob, msg):
    opts = _lib.RpaOptions(sm_scale=1.0, **knob)
    # distinct fake pointers, never dereferenced: the options are checked before any launch
    ptrs = [ctypes.c_void_p(256 * (i + 1)) for i in range(9)]
    rc = lib.rpa_ragged_paged_attention(ctypes.byref(_shape()), ctypes.byref(opts), *ptrs, 0, None)
    assert rc == -1 and msg in lib.rpa_last_error()


def test_null_pointers_rejected(lib):
    rc = lib.rpa_ragged_paged_attention(ctypes.byref(_shape()), None, *([None] * 9), 0, None)
    assert rc == -1 and b"options" in lib.rpa_last_error()
    opts = _lib.RpaOptions(sm_scale=1.0)
    rc = lib.rpa_ragged_paged_attention(ctypes.byref(_shape()), ctypes.byref(opts), *([None] * 9), 0, None)
    assert rc == -1 and b"NULL" in lib.rpa_last_error()


def test_schedule_math_host_checker(tmp_path):
    exe = tmp_path / "sched_check"
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{ROOT / 'tpu-cake_amd' / 'csrc'}",
                    str(ROOT / "tests" / "sched_check.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and out.stdout.startswith("OK"), out.stdout + out.stderr


def test_ctypes_signatures_match_the_header():
    """Every declared entry point's ctypes argtypes count equals its C parameter count
    (an undeclared trailing argument would be marshalled as a C int)."""
    import re
    text = HEADER.read_text()
    lib = _lib.load()
    for name in declared_functions():
        m = re.search(r"\b" + name + r"\s*\(([^)]*)\)", text)
        params = [x for x in m.group(1).split(",") if x.strip() and x.strip() != "void"]
        assert len(getattr(lib, name).argtypes) == len(params), name


def _v1_shape(**kw):
    base = dict(num_seqs=4, num_q_heads=4, num_kv_heads=4, head_dim=32, total_pages=32, page_size=16,
                pages_per_seq=8, bias_len=128)
    base.update(kw)
    return _lib.RpaInklingShape(**base)


@pytest.mark.parametrize("bad,msg", [(dict(num_q_heads=6, num_kv_heads=4), b"divide evenly"),
                                     (dict(head_dim=160), b"head_dim"),
                                     (dict(page_size=0), b"page counts"),
                                     (dict(bias_len=0), b"bias_len")])
def test_v1_invalid_shapes_rejected_before_launch(lib, bad, msg):
    rc = lib.rpa_inkling_decode(ctypes.byref(_v1_shape(**bad)), 1.0, *([None] * 8), 0, None)
    assert rc != 0 and msg in lib.rpa_last_error()
    assert lib.rpa_inkling_workspace_size(ctypes.byref(_v1_shape(**bad))) == 0


def test_v1_null_pointers_rejected(lib):
    rc = lib.rpa_inkling_decode(ctypes.byref(_v1_shape()), 1.0, *([None] * 8), 0, None)
    assert rc == -1 and b"NULL" in lib.rpa_last_error()


class _ShapeCase:
    """A host case with the shapes of a configuration and no data (zero-stride arrays): all that
    rpa_attention_grid reads."""

    def __init__(self, T, hq, hkv, n, pps=128, page=64, pages=4000, kv_dtype="bf16"):
        import numpy as np
        self.q = np.broadcast_to(np.zeros((1, 1, 1), np.uint16), (T, hq, 128))
        self.kv_pages = np.broadcast_to(np.zeros((1, 1, 1, 1), np.uint16), (pages, page, 2 * hkv, 128))
        self.page_indices = np.broadcast_to(np.zeros((1, 1), np.int32), (n, pps))
        self.sm_scale = 128 ** -0.5
        self.kv_dtype = kv_dtype


@pytest.mark.parametrize("case,knobs,expect", [
    # decode batch (C2 shapes): 8-wave workgroups, one per CU; waves_per_cu caps the waves in all
    (dict(T=64, hq=32, hkv=8, n=64), {}, (256, 8)),
    (dict(T=64, hq=32, hkv=8, n=64), {"waves_per_cu": 8}, (256, 8)),
    (dict(T=64, hq=32, hkv=8, n=64), {"waves_per_cu": 7}, (224, 8)),
    (dict(T=64, hq=32, hkv=8, n=64), {"waves_per_cu": 4}, (128, 8)),
    (dict(T=64, hq=32, hkv=8, n=64), {"waves_per_cu": 1}, (32, 8)),
    (dict(T=64, hq=32, hkv=8, n=64, kv_dtype="fp8"), {"waves_per_cu": 6}, (192, 8)),
    # mixed batch (C3 shapes): the co-resident layout, two 4-wave workgroups per CU
    (dict(T=2072, hq=32, hkv=8, n=28), {}, (512, 4)),
    (dict(T=2072, hq=32, hkv=8, n=28), {"waves_per_cu": 4}, (256, 4)),
    (dict(T=2072, hq=32, hkv=8, n=28), {"prefill_tiles": 3}, (256, 8)),
    (dict(T=2072, hq=32, hkv=8, n=28), {"prefill_tiles": -1}, (256, 8)),
    (dict(T=2072, hq=32, hkv=8, n=28, page=16), {}, (256, 8)),  # page 16: no co-resident layout
    # two kv heads (C1 shapes): 2-wave workgroups, four per CU
    (dict(T=4, hq=8, hkv=2, n=4, page=16), {}, (1024, 2)),
    (dict(T=4, hq=8, hkv=2, n=4, page=16), {"waves_per_cu": 4}, (512, 2)),
    (dict(T=4, hq=8, hkv=2, n=4, page=16), {"waves_per_cu": 1}, (128, 2)),
])
def test_attention_grid_rule(lib, case, knobs, expect):
    from tpu_cake_amd import ops
    assert ops.attention_grid(_ShapeCase(**case), knobs, cus=256) == expect


def test_search_refuses_noop_waves_per_cu_candidate():
    from tpu_cake_amd import ops, search
    case = _ShapeCase(T=64, hq=32, hkv=8, n=64)
    grid = lambda c, k: ops.attention_grid(c, k, cus=256)  # noqa: E731
    c = search.SearchContract(config="c2", baseline="base", candidates=(("base", {}), ("w8", {"waves_per_cu": 8})), rounds=4)
    with pytest.raises(ValueError, match="RPA_SEARCH_NOOP_CANDIDATE"):
        search.refuse_noop_candidates(c, case, grid)
    ok = search.SearchContract(config="c2", baseline="base", candidates=(("base", {}), ("w4", {"waves_per_cu": 4})), rounds=4)
    search.refuse_noop_candidates(ok, case, grid)


def test_product_library_has_no_timeline(lib):
    # the product build records no timeline: its read entry point says so without touching a GPU
    import ctypes

    buf = (ctypes.c_int64 * 16)()
    assert lib.rpa_timeline_read(buf, 1, None) == -2  # RPA_E_UNSUPPORTED
    assert b"RPA_TIMELINE" in lib.rpa_last_error()


def test_host_checks_still_see_nan(lib):
    # the device code is built assuming no NaN operands; the host-side option checks are not, and
    # reject a NaN prefill_cost before anything touches a GPU
    import ctypes
    import math

    from tpu_cake_amd import _lib

    shape = _lib.RpaShape(64, 32, 8, 128, 100, 64, 64, 128, _lib.RPA_KV_BF16)
    for cost, ok in ((math.nan, False), (0.45, True), (-math.inf, False)):
        opts = _lib.RpaOptions(sm_scale=0.088, waves_per_cu=0, prefill_tiles=0, prefill_cost=cost)
        grid, waves = ctypes.c_int32(0), ctypes.c_int32(0)
        rc = lib.rpa_attention_grid(ctypes.byref(shape), ctypes.byref(opts), 256, ctypes.byref(grid),
                                    ctypes.byref(waves))
        assert (rc == 0) == ok, (cost, rc, lib.rpa_last_error())
        if not ok:
            assert b"prefill_cost" in lib.rpa_last_error()

"""The attention kernel's timeline (tpu_cake_amd.timeline): the summary of synthetic rows on the CPU,
and on the GPU the tool run end to end through the -DRPA_TIMELINE library variant."""

import os
import pathlib
import subprocess
import sys

import pytest

from tpu_cake_amd import timeline

ROOT = pathlib.Path(__file__).resolve().parent.parent


def _row(**kw):
    r = dict.fromkeys(timeline.FIELDS, 0)
    r.update(kw)
    return r


def test_summary_of_synthetic_rows():
    # 4 workgroups on 2 CUs: 0 and 2 stream-K then joining, 1 and 3 prefill-first
    rows = []
    for b in range(4):
        base = 1000 + 10 * b
        if b % 2 == 0:
            rows.append(_row(start=base, sched=base + 100, first=base + 300, dec=base + 5000, tiles0=base + 5000,
                             ranked=base + 5100, end=base + 8000, role=6, units=7, ntiles=1, nsteps=20, queue=50,
                             setup=200, loop=2000, write=100, where=(b % 8) << 32 | (b // 2) << 8))
        else:
            rows.append(_row(start=base, sched=base + 100, tiles0=base + 100, ranked=base + 400, end=base + 9000,
                             role=1, ntiles=2, nsteps=50, queue=200, setup=600, loop=8000, write=300,
                             where=(b % 8) << 32 | ((b - 1) // 2) << 8))
    text = "\n".join(timeline.summarize(rows, 4, 4, 95.0))
    assert "timeline span (first start to last exit) 90.30 us" in text
    assert "stream-K workgroups with a range: 2; units per range median 7" in text
    assert "first unit's loads issued: median 3.10 us" in text
    # 140 steps in 200 us of loops; the prefill-first pair: 160 us / 100 steps, 4 tiles
    assert "3 tiles" not in text and "6 tiles (or tile parts), 140 chunk steps" in text
    assert "step loop: 1.429 us per step" in text
    assert "prefill-first: 1.600 us per step; per tile: set-up 3.00 us, queue fetch 1.00 us, row writes 1.50 us" in text
    assert "joining: 1.000 us per step" in text
    assert "workgroup b on XCD b mod 8 for 4 of 4" in text
    assert "b and b + 2 on one CU" in text and "for 0 of 2 pairs" in text


@pytest.mark.gpu
def test_timeline_tool_runs_on_c3(cuda, tmp_path):
    lib = ROOT / "tpu-cake_amd" / "tpu_cake_amd" / "librpa_timeline.so"
    if not lib.exists():
        pytest.fail(f"{lib} missing: build with python -m tpu_cake_amd.build")
    print("[case] timeline tool, c3", flush=True)
    env = dict(os.environ, PYTHONPATH=str(ROOT / "tpu-cake_amd"))
    res = subprocess.run([sys.executable, "-m", "tpu_cake_amd.timeline", "--config", "c3", "--runs", "2",
                          "--write", str(tmp_path / "t.md")], env=env, cwd=ROOT, capture_output=True, text=True,
                         timeout=240)
    print(res.stdout[-3000:], res.stderr[-2000:])
    assert res.returncode == 0
    text = (tmp_path / "t.md").read_text()
    assert "prefill tiles: 512 tiles" in text  # C3's 4 chunks x 16 token blocks x 8 kv heads, none split
    assert "stream-K workgroups with a range" in text

"""Build ``librpa.so`` for gfx950 in-tree with hipcc (``python -m tpu_cake_amd.build``).

Also builds ``librpa_timeline.so``: the same sources with ``-DRPA_TIMELINE``, whose attention
kernel records a per-workgroup timeline (read by ``tpu_cake_amd.timeline``); the product path
never loads it.
"""

from __future__ import annotations

import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent.parent
CSRC = PKG.parent / "csrc"
INCLUDE = ROOT / "include"
SOURCES = [CSRC / "rpa_kernels.hip"]
HEADERS = [CSRC / "rpa_schedule.h", INCLUDE / "rpa.h"]
OUTPUT = PKG / "librpa.so"
TIMELINE_OUTPUT = PKG / "librpa_timeline.so"
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def command(output: pathlib.Path = OUTPUT, extra: list[str] | None = None) -> list[str]:
    return [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        # packed fp32 VALU ops are kept out of generated code on this platform
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # device code only: no NaN operands, so fmaxf needs no quieting v_max_f32 x, x before each
        # use (infinities keep their meaning: masked scores are -inf); host-side checks keep NaN
        "-Xarch_device", "-fno-honor-nans",
        f"-I{INCLUDE}", f"-I{CSRC}", *(extra or []),
        *[str(s) for s in SOURCES], "-o", str(output),
    ]


def _start(output: pathlib.Path, extra: list[str]):
    tmp = output.with_suffix(".so.tmp")
    cmd = command(tmp, extra)
    return output, tmp, cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)


def _finish(job, verbose: bool) -> pathlib.Path:
    output, tmp, cmd, proc = job
    _, err = proc.communicate()
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, output)
    return output


def build(verbose: bool = False, timeline: bool = True) -> pathlib.Path:
    """Compile every HIP source into ``librpa.so`` (always recompiles), and (``timeline``) the
    timeline variant beside it, the two compilations in parallel.  Returns the product path."""
    jobs = [_start(OUTPUT, [])]
    if timeline:
        jobs.append(_start(TIMELINE_OUTPUT, ["-DRPA_TIMELINE"]))
    out = [_finish(j, verbose) for j in jobs]
    return out[0]


if __name__ == "__main__":
    print(build(verbose=True))

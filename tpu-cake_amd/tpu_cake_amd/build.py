"""Build ``librpa.so`` for gfx950 in-tree with hipcc (``python -m tpu_cake_amd.build``)."""

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
        f"-I{INCLUDE}", f"-I{CSRC}", *(extra or []),
        *[str(s) for s in SOURCES], "-o", str(output),
    ]


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every HIP source into ``librpa.so`` (always recompiles)."""
    tmp = OUTPUT.with_suffix(".so.tmp")
    cmd = command(tmp)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{res.stderr}")
    if verbose and res.stderr.strip():
        print(res.stderr, file=sys.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose=True))

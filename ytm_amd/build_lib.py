"""Builds libytm.so (the HIP kernels + C-ABI) for gfx950, in-tree next to this file.

    python -m ytm_amd.build_lib
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
SOURCES = [HERE / "csrc" / "ytm_kernels.hip", HERE / "csrc" / "ytm_api.hip"]
OUT = HERE / "libytm.so"

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "--offload-arch=gfx950",
    # exact IEEE semantics for the parity-critical float/double compares and updates
    "-ffp-contract=off",
    # packed-fp32 VALU forms off
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def build(verbose: bool = False) -> Path:
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-o", str(tmp), *map(str, SOURCES)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    if verbose and res.stderr:
        print(res.stderr, file=sys.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))

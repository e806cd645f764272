"""Ahead-of-time build of liborigami_layout.so (HIP, gfx950).

The library is built in-tree (origami_amd/_lib/) so that it ships with the
package; nothing is JIT-compiled at import time.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
SOURCES = [PKG / "csrc" / "origami_layout.hip", PKG / "csrc" / "origami_dequant.hip"]
INCLUDE = REPO / "include"
LIB_DIR = PKG / "_lib"
LIB_PATH = LIB_DIR / "liborigami_layout.so"
ARCH = os.environ.get("ORIGAMI_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    # no implicit contraction: float results round exactly where the source
    # rounds (fused multiply-adds are written out as fmaf)
    "-ffp-contract=off",
    # packed FP32 VALU forms are disabled for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; ROCm is required to build liborigami_layout.so")


def build(verbose: bool = False) -> Path:
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", *map(str, SOURCES), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

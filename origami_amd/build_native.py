"""Ahead-of-time build of liborigami_layout.so (HIP, gfx950) and of the
PyTorch-ROCm extension module origami_bitpack_hip over its C ABI.

Both are built in-tree (origami_amd/_lib/) so that they ship with the
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
EXT_NAME = "origami_bitpack_hip"
EXT_SOURCE = PKG / "csrc" / "origami_torch_ext.cpp"
EXT_PATH = LIB_DIR / f"{EXT_NAME}.so"
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


def build_library(verbose: bool = False) -> Path:
    """Compiles each HIP source to an object (in parallel; no device code is
    shared between them), then links the shared library."""
    from concurrent.futures import ThreadPoolExecutor

    LIB_DIR.mkdir(parents=True, exist_ok=True)
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(exist_ok=True)
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    jobs = []
    for src in SOURCES:
        obj = obj_dir / (src.stem + ".o")
        jobs.append([hipcc(), *compile_flags, f"-I{INCLUDE}", "-c", str(src), "-o", str(obj)])
    for cmd in jobs if verbose else ():
        print(" ".join(cmd), flush=True)
    with ThreadPoolExecutor(max_workers=len(jobs)) as pool:
        for fut in [pool.submit(subprocess.run, cmd, check=True) for cmd in jobs]:
            fut.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    link = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *[j[-1] for j in jobs],
            "-o", str(tmp)]
    if verbose:
        print(" ".join(link), flush=True)
    subprocess.run(link, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def build_extension(verbose: bool = False) -> Path:
    """The torch extension: host C++ only (g++), linked to liborigami_layout.so
    next to it (rpath $ORIGIN) and to torch's libraries."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    includes = [*cpp_extension.include_paths(device_type="cuda"), sysconfig.get_paths()["include"],
                str(INCLUDE), f"{rocm}/include"]
    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch.compiled_with_cxx11_abi())
    tmp = EXT_PATH.with_suffix(".so.tmp")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           *[f"-I{d}" for d in includes], str(EXT_SOURCE), "-o", str(tmp),
           f"-L{LIB_DIR}", "-lorigami_layout", f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch",
           "-ltorch_cpu", "-ltorch_hip", "-ltorch_python", "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, EXT_PATH)
    return EXT_PATH


def build(verbose: bool = False) -> Path:
    """Builds the library, then the extension module over it."""
    build_library(verbose)
    build_extension(verbose)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

"""Loader of origami_bitpack_hip, the PyTorch-ROCm extension module built
in-tree over liborigami_layout.so (origami_amd/csrc/origami_torch_ext.cpp).

It exports the reference extension's function names
(bitpack_layout_cuda.cpp:894-903) and the fused paths; the hot calls of
lossless/native_gpu.py go through it.  There is no CPU fallback: if the
module is not built, every call raises.
"""
from __future__ import annotations

import importlib.machinery
import importlib.util
import threading
from pathlib import Path
from types import ModuleType

EXT_NAME = "origami_bitpack_hip"
EXT_PATH = Path(__file__).resolve().parent / "_lib" / f"{EXT_NAME}.so"

_mod: ModuleType | None = None
_lock = threading.Lock()


def ext() -> ModuleType:
    """The extension module, loaded once; raises RuntimeError if not built."""
    global _mod
    if _mod is not None:
        return _mod
    with _lock:
        if _mod is None:
            if not EXT_PATH.exists():
                raise RuntimeError(
                    f"{EXT_PATH} is not built; run `python -m origami_amd.build_native` "
                    "(the Origami HIP layout path has no CPU fallback)")
            import torch  # noqa: F401 - the module links against torch's libraries

            loader = importlib.machinery.ExtensionFileLoader(EXT_NAME, str(EXT_PATH))
            spec = importlib.util.spec_from_file_location(EXT_NAME, str(EXT_PATH), loader=loader)
            mod = importlib.util.module_from_spec(spec)
            loader.exec_module(mod)
            from origami_amd import _native

            if mod.abi_version() != _native.ABI_VERSION:
                raise RuntimeError(f"{EXT_NAME} was built against another ABI; rebuild it")
            _mod = mod
    return _mod

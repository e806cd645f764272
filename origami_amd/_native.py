"""ctypes binding of liborigami_layout.so (the C ABI in include/origami_layout.h).

This is the only place Python touches the native library.  There is no CPU
fallback: if the library is missing, every call raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "liborigami_layout.so"
ABI_VERSION = 3

ORIGAMI_OK = 0
ORIGAMI_ERR_INVALID = 1
ORIGAMI_ERR_UNSUPPORTED = 2
ORIGAMI_ERR_HIP = 3

CACHE_KV_FIRST = 0
CACHE_BLOCKS_FIRST = 1

DTYPE_FLOAT16 = 1
DTYPE_BFLOAT16 = 2
DTYPE_FLOAT32 = 3

KIVI_PACKED_LSB = 0
KIVI_NIBBLE3 = 1

_i64 = ctypes.c_int64
_p = ctypes.c_void_p

# name -> argument types (return type is int for all but origami_last_error)
_SIGNATURES: dict[str, list] = {
    "origami_abi_version": [],
    "origami_set_rows_grid_limit": [_i64],
    "origami_validate_chunks": [_p, _p, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64],
    "origami_plan_planes": [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "origami_unpack_canonical_storage_chunks": [
        _p, _i64, _p, _p, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _p, _i64, _p],
    "origami_pack_canonical_storage_chunks": [
        _p, _i64, _p, _p, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _p, _i64, _p],
    "origami_unpack_canonical_to_kv_cache": [
        _p, _i64, _p, _p, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "origami_unpack_canonical_to_kv_cache_noalloc": [
        _p, _i64, _p, _p, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "origami_restore_plan_create": [
        _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "origami_restore_plan_launch": [_p, _p, _i64, _p, _p],
    "origami_unpack_canonical_to_kv_cache_batch": [
        _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p],
    "origami_pack_canonical_from_kv_cache": [
        _p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _i64, _p, _i64, _p],
    "origami_scatter_kv_blocks": [_p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "origami_gather_kv_blocks": [_p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p, _p],
    "origami_cachegen_unpack_dequantize_to_kv_cache": [
        _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64,
        _p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _p],
    "origami_cachegen_unpack_dequantize": [
        _p, _i64, _p, _p, _p, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "origami_kivi_dequantize_to_kv_cache": [
        _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p,
        _i64, _p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _p],
}

EXPORTED_SYMBOLS = ("origami_last_error", "origami_restore_plan_destroy",
                    "origami_debug_counters", *_SIGNATURES)

_lib: ctypes.CDLL | None = None
_lock = threading.Lock()


class OrigamiNativeError(RuntimeError):
    """A failing call into liborigami_layout.so (carries the status code)."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


def lib() -> ctypes.CDLL:
    """Loads the library once; raises RuntimeError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python -m origami_amd.build_native`"
                    " (the Origami HIP layout path has no CPU fallback)")
            L = ctypes.CDLL(str(LIB_PATH))
            L.origami_last_error.restype = ctypes.c_char_p
            L.origami_last_error.argtypes = []
            for name, args in _SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = ctypes.c_int
                fn.argtypes = args
            L.origami_set_rows_grid_limit.restype = ctypes.c_int64
            L.origami_restore_plan_destroy.restype = None
            L.origami_restore_plan_destroy.argtypes = [_p]
            L.origami_debug_counters.restype = None
            L.origami_debug_counters.argtypes = [_p, _p]
            if L.origami_abi_version() != ABI_VERSION:
                raise RuntimeError("liborigami_layout.so ABI version mismatch; rebuild it")
            _lib = L
    return _lib


_entry_points: dict = {}


def call(name: str, *args) -> int:
    """Calls an entry point; raises OrigamiNativeError on a non-zero status."""
    L = lib()
    entry = _entry_points.get(name)
    if entry is None or entry[0] is not L:  # first call, or the library was reloaded
        entry = _entry_points[name] = (L, getattr(L, name))
    rc = entry[1](*args)
    if rc != ORIGAMI_OK:
        msg = L.origami_last_error().decode(errors="replace")
        raise OrigamiNativeError(rc, msg)
    return rc


def host_ptr(arr: np.ndarray) -> int:
    """Address of a C-contiguous host array (the caller keeps it alive)."""
    assert arr.flags.c_contiguous
    return arr.ctypes.data


def i64_array(values) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(values, dtype=np.int64))


def set_rows_grid_limit(max_workgroups: int) -> int:
    """Caps row-kernel workgroups for launches on this thread; returns the old cap."""
    return int(lib().origami_set_rows_grid_limit(int(max_workgroups)))


def debug_counters() -> tuple[int, int]:
    """(chunk plans created, device allocations made) by the library so far."""
    plans, allocs = ctypes.c_int64(0), ctypes.c_int64(0)
    lib().origami_debug_counters(ctypes.byref(plans), ctypes.byref(allocs))
    return int(plans.value), int(allocs.value)

"""numpy/ctypes front end of the CPU oracle (oracle/layout_oracle.c and
oracle/dequant_oracle.c).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, by __graft_entry__.smoke() as
the checker, and by bench.py's cpu_baseline leg as the timed CPU baseline.
The product package (origami_amd) never imports this module.

Arrays are numpy; byte tensors are uint8, metadata int64.  Axis positions
follow the reference's convention [token_axis, head_axis, head_dim_axis,
layer_axis or -1] (lossless/native_cpu.py:120-130).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "_build" / "liborigami_oracle.so"
_lib = None

_u8p = ctypes.POINTER(ctypes.c_uint8)
_i64p = ctypes.POINTER(ctypes.c_int64)


def build(force: bool = False) -> Path:
    """Compile the oracle with gcc (via oracle/Makefile)."""
    if force or not LIB_PATH.exists():
        subprocess.run(["make", "-s"] + (["-B"] if force else []) + ["-C", str(_HERE)],
                       check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.oracle_last_error.restype = ctypes.c_char_p
        L.oracle_unpack_symbol.restype = ctypes.c_uint8
        L.oracle_unpack_symbol.argtypes = [_u8p, ctypes.c_int64, ctypes.c_int64,
                                           ctypes.c_int]
        L.oracle_unpack_canonical.argtypes = [
            _u8p, _i64p, _i64p, _i64p, ctypes.c_int64, _i64p, ctypes.c_int,
            _i64p, _u8p, ctypes.c_int64]
        L.oracle_pack_canonical.argtypes = [
            _u8p, ctypes.c_int64, _i64p, _i64p, _i64p, ctypes.c_int64, _i64p,
            ctypes.c_int, _i64p, _u8p, ctypes.c_int64]
        L.oracle_scatter_kv_cache.argtypes = [
            _u8p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _i64p,
            ctypes.c_int64, _u8p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int]
        L.oracle_gather_kv_cache.argtypes = [
            _u8p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_int, _i64p, ctypes.c_int64, _u8p]
        L.oracle_set_threads.argtypes = [ctypes.c_int]
        L.oracle_dequant_last_error.restype = ctypes.c_char_p
        L.oracle_half_to_float.restype = ctypes.c_float
        L.oracle_half_to_float.argtypes = [ctypes.c_uint16]
        L.oracle_float_to_half.restype = ctypes.c_uint16
        L.oracle_float_to_half.argtypes = [ctypes.c_float]
        L.oracle_float_to_bf16.restype = ctypes.c_uint16
        L.oracle_float_to_bf16.argtypes = [ctypes.c_float]
        _v, _i, _c = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.oracle_cachegen_to_kv_cache.argtypes = [
            _u8p, _i, _i, _i, _i, _i, _c, _c, _i, _i, _v, _v, _c, _v, _c, _c, _i, _i, _i64p,
            _i, _i, _i, _i]
        L.oracle_cachegen_unpack_dequantize.argtypes = [
            _u8p, _i, _i64p, _i64p, _i64p, _i64p, _i, _v, _v, _c, _i, _i, _i, _v]
        L.oracle_kivi_to_kv_cache.argtypes = [
            _u8p, _i, _i, _i, _i, _i, _c, _c, _i, _i, _v, _v, _v, _v, _v, _v, _c, _v, _c, _c,
            _i, _i, _i64p, _i, _i, _i, _i]
        _lib = L
    return _lib


def _p8(a: np.ndarray):
    assert a.dtype == np.uint8 and a.flags.c_contiguous
    return a.ctypes.data_as(_u8p)


def _p64(a: np.ndarray):
    assert a.dtype == np.int64 and a.flags.c_contiguous
    return a.ctypes.data_as(_i64p)


def _i64(values) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(values, dtype=np.int64))


def _check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(lib().oracle_last_error().decode())


def set_threads(n: int) -> None:
    lib().oracle_set_threads(int(n))


def max_threads() -> int:
    return int(lib().oracle_max_threads())


def chunk_offsets(specs, bits) -> np.ndarray:
    """Byte offsets [N+1]: chunk k holds ceil(n_k*b_k/8) bytes (cpp:181-185)."""
    specs = _i64(specs).reshape(-1, 6)
    bits = np.broadcast_to(_i64(bits), (specs.shape[0],))
    n = ((specs[:, 1] - specs[:, 0]) * (specs[:, 3] - specs[:, 2])
         * (specs[:, 5] - specs[:, 4]))
    sizes = (n * bits + 7) // 8
    return np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)


def unpack_symbol(src: np.ndarray, index: int, bits: int) -> int:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    return int(lib().oracle_unpack_symbol(_p8(src), src.size, int(index), int(bits)))


def unpack_canonical(flat, offsets, bits, specs, shape, axes) -> np.ndarray:
    flat = np.ascontiguousarray(flat, dtype=np.uint8)
    specs = _i64(specs).reshape(-1, 6)
    n = specs.shape[0]
    bits = _i64(np.broadcast_to(_i64(bits), (n,)))
    offsets, shape, axes = _i64(offsets), _i64(shape), _i64(axes)
    out = np.empty(int(np.prod(shape)), dtype=np.uint8)
    _check(lib().oracle_unpack_canonical(
        _p8(flat), _p64(offsets), _p64(bits), _p64(specs), n, _p64(shape),
        shape.size, _p64(axes), _p8(out), out.size))
    return out


def pack_canonical(symbols, bits, specs, shape, axes):
    """Returns (flat stream, offsets[N+1])."""
    symbols = np.ascontiguousarray(symbols, dtype=np.uint8).reshape(-1)
    specs = _i64(specs).reshape(-1, 6)
    n = specs.shape[0]
    bits = _i64(np.broadcast_to(_i64(bits), (n,)))
    offsets = chunk_offsets(specs, bits)
    shape, axes = _i64(shape), _i64(axes)
    flat = np.zeros(int(offsets[-1]), dtype=np.uint8)
    _check(lib().oracle_pack_canonical(
        _p8(symbols), symbols.size, _p64(offsets), _p64(bits), _p64(specs), n,
        _p64(shape), shape.size, _p64(axes), _p8(flat), flat.size))
    return flat, offsets


def scatter_kv_cache(value, tokens, heads, head_bytes, block_ids, cache,
                     blocks_first: bool = False) -> None:
    """value: uint8 bytes of [2, tokens, heads, head_bytes]; cache modified in place."""
    value = np.ascontiguousarray(value, dtype=np.uint8).reshape(-1)
    assert value.size == 2 * tokens * heads * head_bytes
    ids = _i64(block_ids)
    assert cache.dtype == np.uint8 and cache.flags.c_contiguous
    if blocks_first:
        NB, bs = cache.shape[0], cache.shape[2]
    else:
        NB, bs = cache.shape[1], cache.shape[2]
    _check(lib().oracle_scatter_kv_cache(
        _p8(value), int(tokens), int(heads), int(head_bytes), _p64(ids), ids.size,
        _p8(cache), int(NB), int(bs), int(bool(blocks_first))))


def gather_kv_cache(cache, block_ids, blocks_first: bool = False) -> np.ndarray:
    """cache: uint8 [2,NB,bs,H,C] or [NB,2,bs,H,C]; returns bytes of [2, nblk*bs, H, C]."""
    assert cache.dtype == np.uint8 and cache.flags.c_contiguous and cache.ndim == 5
    if blocks_first:
        NB, _, bs, H, C = cache.shape
    else:
        _, NB, bs, H, C = cache.shape
    ids = _i64(block_ids)
    out = np.empty(2 * ids.size * bs * H * C, dtype=np.uint8)
    _check(lib().oracle_gather_kv_cache(
        _p8(cache), int(NB), int(bs), int(H), int(C), int(bool(blocks_first)),
        _p64(ids), ids.size, _p8(out)))
    return out


def restore_layer(flat, offsets, bits, specs, tokens, heads, head_bytes,
                  block_ids, cache, blocks_first: bool = False) -> None:
    """Unpack a layer stream in the [2T, H, C] token/head/head_dim symbol
    layout, then scatter it into the paged cache (the full restore path)."""
    symbols = unpack_canonical(flat, offsets, bits, specs,
                               [2 * tokens, heads, head_bytes], [0, 1, 2, -1])
    scatter_kv_cache(symbols, tokens, heads, head_bytes, block_ids, cache,
                     blocks_first)


__all__ = [
    "build", "lib", "set_threads", "max_threads", "chunk_offsets",
    "unpack_symbol", "unpack_canonical", "pack_canonical", "scatter_kv_cache",
    "gather_kv_cache", "restore_layer", "LIB_PATH",
]

if os.environ.get("ORIGAMI_ORACLE_AUTOBUILD", "1") == "1" and not LIB_PATH.exists():
    try:
        build()
    except Exception:  # built on demand by lib() again, which raises if it cannot
        pass


# ---------------------------------------------------------------------------
# Fused dequantize paths (dequant_oracle.c)
# ---------------------------------------------------------------------------

def _dq_check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(lib().oracle_dequant_last_error().decode())


def half_to_float(bits: int) -> float:
    return float(lib().oracle_half_to_float(int(bits)))


def float_to_half(x: float) -> int:
    return int(lib().oracle_float_to_half(float(x)))


def float_to_bf16(x: float) -> int:
    return int(lib().oracle_float_to_bf16(float(x)))


def _meta(a: np.ndarray) -> tuple[np.ndarray, int]:
    """float16 arrays travel as their bits; float32 as is."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        return a.view(np.uint16), 1
    if a.dtype == np.float32:
        return a, 0
    raise TypeError("metadata must be float16 or float32")


def _vp(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


def cachegen_to_kv_cache(bytestream, key_offset, key_bytes, value_offset, value_bytes,
                         key_bits, value_bits, key_bins, value_bins, max_key, max_value,
                         cache: np.ndarray, out_is_bf16: bool, blocks_first: bool, block_ids,
                         tokens: int, heads: int, head_dim: int) -> None:
    """In place on `cache` (uint16 bits of float16 / bfloat16, rank 5)."""
    stream = np.ascontiguousarray(bytestream, dtype=np.uint8).reshape(-1)
    mk, half = _meta(max_key)
    mv, half_v = _meta(max_value)
    assert half == half_v
    ids = _i64(block_ids)
    assert cache.dtype == np.uint16 and cache.flags.c_contiguous and cache.ndim == 5
    nb = cache.shape[0] if blocks_first else cache.shape[1]
    _dq_check(lib().oracle_cachegen_to_kv_cache(
        _p8(stream), stream.size, int(key_offset), int(key_bytes), int(value_offset),
        int(value_bytes), int(key_bits), int(value_bits), int(key_bins), int(value_bins),
        _vp(mk), _vp(mv), half, _vp(cache), int(bool(out_is_bf16)), int(bool(blocks_first)),
        int(nb), int(cache.shape[2]), _p64(ids), ids.size, int(tokens), int(heads),
        int(head_dim)))


def cachegen_unpack_dequantize(bytestream, offsets, bits_per_layer, key_bins, value_bins,
                               max_key, max_value, tokens: int, heads: int,
                               head_dim: int) -> np.ndarray:
    """Returns float16 [layers, 2, heads, tokens, head_dim]."""
    stream = np.ascontiguousarray(bytestream, dtype=np.uint8).reshape(-1)
    offs, bits = _i64(offsets), _i64(bits_per_layer)
    kb, vb = _i64(key_bins), _i64(value_bins)
    layers = bits.size // 2
    mk, half = _meta(max_key)
    mv, _ = _meta(max_value)
    out = np.zeros((layers, 2, heads, tokens, head_dim), dtype=np.uint16)
    _dq_check(lib().oracle_cachegen_unpack_dequantize(
        _p8(stream), stream.size, _p64(offs), _p64(bits), _p64(kb), _p64(vb), layers,
        _vp(mk), _vp(mv), half, int(tokens), int(heads), int(head_dim), _vp(out)))
    return out.view(np.float16)


def kivi_to_kv_cache(bytestream, key_offset, key_bytes, value_offset, value_bytes, bits,
                     nibble3: bool, group_size, sink_tokens, key_scale, key_zero, value_scale,
                     value_zero, key_sink, value_sink, cache: np.ndarray, out_is_bf16: bool,
                     blocks_first: bool, block_ids, tokens: int, heads: int,
                     head_dim: int) -> None:
    """In place on `cache` (uint16 bits of float16 / bfloat16, rank 5)."""
    stream = np.ascontiguousarray(bytestream, dtype=np.uint8).reshape(-1)
    metas = [_meta(a) for a in (key_scale, key_zero, value_scale, value_zero, key_sink,
                                value_sink)]
    half = metas[0][1]
    assert all(m[1] == half for m in metas)
    ids = _i64(block_ids)
    assert cache.dtype == np.uint16 and cache.flags.c_contiguous and cache.ndim == 5
    nb = cache.shape[0] if blocks_first else cache.shape[1]
    _dq_check(lib().oracle_kivi_to_kv_cache(
        _p8(stream), stream.size, int(key_offset), int(key_bytes), int(value_offset),
        int(value_bytes), int(bits), int(bool(nibble3)), int(group_size), int(sink_tokens),
        *[_vp(m[0]) for m in metas], half, _vp(cache), int(bool(out_is_bf16)),
        int(bool(blocks_first)), int(nb), int(cache.shape[2]), _p64(ids), ids.size,
        int(tokens), int(heads), int(head_dim)))

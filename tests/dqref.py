"""Independent restatements of the reference's unfused dequantize paths, used
to pin the dequant oracle (oracle/dequant_oracle.c) and to build test inputs.

Written from the reference's Python adapters, not from the oracle's C code:

* CacheGen (quantization/cachegen_adapter.py:117-142, 364-370, 880-919): the
  K/V streams are a linear LSB-first pack of the [tokens, C] symbols
  (tests/bitref.py); a value is `(q.float() - c) / c * max` with torch
  float32 tensor ops, c = bins // 2 - 1; the result is stacked to
  [2, tokens, heads, head_dim], cast with `.to(dtype)` and assigned block by
  block into the paged cache.
* KIVI (quantization/kivi_adapter.py:28-54, 97-122, 469-531): streams use
  KIVI's own packers (2 and 4 bits LSB-first, 3 bits one symbol per nibble,
  8 bits identity) over the key order head_dim > head > token and the value
  order head > head_dim > token.  The multiply-add `s * scale + zero` is
  evaluated exactly in float64 and rounded once to float32, i.e. a fused
  multiply-add, which is how nvcc compiles the reference kernel's
  expression (bitpack_layout_cuda.cu:651-660); every element is checked to
  be exact in float64 before it is used.
"""
from __future__ import annotations

import numpy as np
import torch

from tests import bitref


# ---------------------------------------------------------------------------
# Streams
# ---------------------------------------------------------------------------

def linear_unpack(stream: np.ndarray, bits: int, count: int) -> np.ndarray:
    """Symbols 0..count-1 of an LSB-first stream; bytes past it read as 0."""
    need = (count * bits + 7) // 8
    buf = np.zeros(need, dtype=np.uint8)
    n = min(need, stream.size)
    buf[:n] = stream[:n]
    return bitref.bits_unpack(buf, bits, count)


def kivi_pack(values: np.ndarray, bits: int) -> np.ndarray:
    """kivi_adapter.py:28-54 (_pack_lowbit_values)."""
    v = np.asarray(values, dtype=np.uint8).reshape(-1)
    if bits == 8:
        return v.copy()
    if bits in (3, 4):
        if v.size % 2:
            v = np.concatenate([v, np.zeros(1, np.uint8)])
        pairs = v.reshape(-1, 2)
        m = np.uint8(0x07 if bits == 3 else 0x0F)
        return ((pairs[:, 0] & m) | ((pairs[:, 1] & m) << 4)).astype(np.uint8)
    if bits == 2:
        pad = (-v.size) % 4
        if pad:
            v = np.concatenate([v, np.zeros(pad, np.uint8)])
        g = v.reshape(-1, 4) & np.uint8(3)
        return (g[:, 0] | (g[:, 1] << 2) | (g[:, 2] << 4) | (g[:, 3] << 6)).astype(np.uint8)
    raise ValueError("KIVI packs 2, 3, 4 or 8 bits")


def kivi_unpack(stream: np.ndarray, bits: int, count: int, nibble3: bool) -> np.ndarray:
    """kivi_adapter.py:57-94 for the KIVI container; LSB-first otherwise."""
    if nibble3 and bits == 3:
        need = (count + 1) // 2
        buf = np.zeros(need, dtype=np.uint8)
        n = min(need, stream.size)
        buf[:n] = stream[:n]
        out = np.empty(need * 2, dtype=np.uint8)
        out[0::2] = buf & 0x07
        out[1::2] = (buf >> 4) & 0x07
        return out[:count]
    return linear_unpack(stream, bits, count)


def kivi_key_order(q_body: np.ndarray, heads: int, head_dim: int) -> np.ndarray:
    """[body, H*D] symbols -> key stream order (d, h, token)."""
    body = q_body.shape[0]
    return np.ascontiguousarray(
        q_body.reshape(body, heads, head_dim).transpose(2, 1, 0)).reshape(-1)


def kivi_value_order(q_body: np.ndarray, heads: int, head_dim: int) -> np.ndarray:
    """[body, H*D] symbols -> value stream order (h, d, token)."""
    body = q_body.shape[0]
    return np.ascontiguousarray(
        q_body.reshape(body, heads, head_dim).transpose(1, 2, 0)).reshape(-1)


# ---------------------------------------------------------------------------
# Paged assignment
# ---------------------------------------------------------------------------

def assign_blocks(cache: torch.Tensor, canonical: torch.Tensor, blocks_first: bool,
                  block_ids, tokens: int) -> None:
    """cache[block] = canonical[kv, block tokens] for valid ids, t < tokens
    (the block assignment of cachegen_adapter.py:913-917, restricted to the
    restored tokens as the fused kernel is)."""
    nb = cache.shape[0] if blocks_first else cache.shape[1]
    bs = cache.shape[2]
    for lb, pid in enumerate(int(b) for b in block_ids):
        if pid < 0 or pid >= nb:
            continue
        t0, t1 = lb * bs, min(lb * bs + bs, tokens)
        if t1 <= t0:
            continue
        for kv in (0, 1):
            dst = cache[pid, kv] if blocks_first else cache[kv, pid]
            dst[: t1 - t0] = canonical[kv, t0:t1]


# ---------------------------------------------------------------------------
# CacheGen
# ---------------------------------------------------------------------------

def cachegen_dequantize_plane(q: np.ndarray, max_abs: np.ndarray, bins: int) -> torch.Tensor:
    """cachegen_adapter.py:364-370 on [tokens, C] symbols and [tokens] maxima."""
    center = bins // 2 - 1
    qt = torch.from_numpy(np.ascontiguousarray(q)).to(torch.float32)
    mx = torch.from_numpy(np.ascontiguousarray(max_abs)).to(torch.float32).reshape(-1, 1)
    return (qt - center) / center * mx


def cachegen_reference_cache(stream: np.ndarray, key_offset: int, key_bytes: int,
                             value_offset: int, value_bytes: int, key_bits: int,
                             value_bits: int, key_bins: int, value_bins: int,
                             max_key: np.ndarray, max_value: np.ndarray, cache: torch.Tensor,
                             blocks_first: bool, block_ids, tokens: int, heads: int,
                             head_dim: int) -> None:
    C = heads * head_dim
    planes = []
    for off, nbytes, bits, bins, mx in ((key_offset, key_bytes, key_bits, key_bins, max_key),
                                        (value_offset, value_bytes, value_bits, value_bins,
                                         max_value)):
        q = linear_unpack(stream[off:off + nbytes], bits, tokens * C).reshape(tokens, C)
        planes.append(cachegen_dequantize_plane(q, mx[:tokens], bins)
                      .reshape(tokens, heads, head_dim))
    canonical = torch.stack(planes, dim=0).to(cache.dtype)
    assign_blocks(cache, canonical, blocks_first, block_ids, tokens)


def cachegen_reference_dense(stream: np.ndarray, offsets, bits_per_layer, key_bins,
                             value_bins, max_key: np.ndarray, max_value: np.ndarray,
                             tokens: int, heads: int, head_dim: int) -> torch.Tensor:
    """float16 [layers, 2, heads, tokens, head_dim]."""
    layers = len(bits_per_layer) // 2
    C = heads * head_dim
    out = torch.empty((layers, 2, heads, tokens, head_dim), dtype=torch.float16)
    for j in range(2 * layers):
        kv, layer = (1, j - layers) if j >= layers else (0, j)
        seg = stream[offsets[j]:offsets[j + 1]]
        q = linear_unpack(seg, int(bits_per_layer[j]), tokens * C).reshape(tokens, C)
        bins = int(value_bins[layer] if kv else key_bins[layer])
        mx = (max_value if kv else max_key).reshape(layers, tokens)[layer]
        v = cachegen_dequantize_plane(q, mx, bins).reshape(tokens, heads, head_dim)
        out[layer, kv] = v.permute(1, 0, 2).to(torch.float16)
    return out


# ---------------------------------------------------------------------------
# KIVI
# ---------------------------------------------------------------------------

def exact_fma32(s: np.ndarray, scale: np.ndarray, zero: np.ndarray) -> np.ndarray:
    """fmaf(s, scale, zero) for float32 inputs, through exact float64."""
    p = s.astype(np.float64) * scale.astype(np.float64)   # exact: <= 8 + 24 bits
    z = zero.astype(np.float64)
    r = p + z
    bp = r - z
    err = (p - bp) + (z - (r - bp))                        # TwoSum error term
    assert np.all(err == 0), "float64 sum not exact; choose smaller exponent spans"
    return r.astype(np.float32)


def kivi_reference_cache(stream: np.ndarray, key_offset: int, key_bytes: int,
                         value_offset: int, value_bytes: int, bits: int, nibble3: bool,
                         group_size: int, sink_tokens: int, key_scale, key_zero, value_scale,
                         value_zero, key_sink, value_sink, cache: torch.Tensor,
                         blocks_first: bool, block_ids, tokens: int, heads: int,
                         head_dim: int) -> None:
    C = heads * head_dim
    body = tokens - sink_tokens
    vgroups = (C + group_size - 1) // group_size
    f32 = lambda a: np.asarray(a).astype(np.float32)  # noqa: E731
    kq = kivi_unpack(stream[key_offset:key_offset + key_bytes], bits, body * C, nibble3)
    vq = kivi_unpack(stream[value_offset:value_offset + value_bytes], bits, body * C, nibble3)
    # stream order -> [body, H, D]
    kq = kq.reshape(head_dim, heads, body).transpose(2, 1, 0).reshape(body, C)
    vq = vq.reshape(heads, head_dim, body).transpose(2, 0, 1).reshape(body, C)
    rows = np.arange(body) // group_size
    cols = np.arange(C) // group_size
    ks = f32(key_scale).reshape(-1, C)[rows]
    kz = f32(key_zero).reshape(-1, C)[rows]
    vs = f32(value_scale).reshape(body, vgroups)[:, cols] if body else np.zeros((0, C), np.float32)
    vz = f32(value_zero).reshape(body, vgroups)[:, cols] if body else np.zeros((0, C), np.float32)
    kb = exact_fma32(kq.astype(np.float32), ks, kz)
    vb = exact_fma32(vq.astype(np.float32), vs, vz)
    k = np.concatenate([f32(key_sink).reshape(sink_tokens, C), kb], axis=0)
    v = np.concatenate([f32(value_sink).reshape(sink_tokens, C), vb], axis=0)
    canonical = torch.from_numpy(np.stack([k, v]).reshape(2, tokens, heads, head_dim)).to(
        cache.dtype)
    assign_blocks(cache, canonical, blocks_first, block_ids, tokens)

"""Independent statements of the canonical format used to pin the oracle.

These are written from the format's definition, not from the oracle's code:
a chunk's symbols are enumerated with numpy fancy indexing in head, channel,
token (fastest) order, and the stream is the concatenation of each symbol's
b bits, least significant bit first, zero-padded to a whole byte
(np.packbits with bitorder="little").
"""
from __future__ import annotations

import numpy as np


def chunk_symbols(sym3: np.ndarray, spec) -> np.ndarray:
    """sym3: [T, H, C] view of the symbol tensor; spec: (hs,he,cs,ce,ts,te)."""
    hs, he, cs, ce, ts, te = (int(x) for x in spec)
    box = sym3[ts:te, hs:he, cs:ce]            # [t, h, c]
    return np.ascontiguousarray(box.transpose(1, 2, 0)).reshape(-1)  # h, c, t fastest


def bits_pack(values: np.ndarray, bits: int) -> np.ndarray:
    v = np.asarray(values, dtype=np.uint8) & np.uint8((1 << bits) - 1)
    # [n, 8] LSB-first bit matrix, keep the low `bits` columns
    mat = np.unpackbits(v[:, None], axis=1, bitorder="little")[:, :bits]
    return np.packbits(mat.reshape(-1), bitorder="little")


def bits_unpack(stream: np.ndarray, bits: int, count: int) -> np.ndarray:
    flat = np.unpackbits(np.asarray(stream, dtype=np.uint8), bitorder="little")
    flat = flat[: count * bits].reshape(count, bits)
    weights = (1 << np.arange(bits)).astype(np.uint32)
    return (flat.astype(np.uint32) @ weights).astype(np.uint8)


def to_tok_head_chan(symbols: np.ndarray, shape, axes) -> np.ndarray:
    """View the flat symbol tensor as [T, H, C] using axis positions."""
    arr = np.asarray(symbols).reshape(shape)
    tok, head, hd, layer = (int(a) for a in axes)
    if layer >= 0:
        arr = arr[(slice(None),) * layer + (0,)]  # a view, not a copy
        tok, head, hd = (a - (1 if a > layer else 0) for a in (tok, head, hd))
    return arr.transpose(tok, head, hd)


def reference_stream(symbols, shape, axes, specs, bits) -> tuple[np.ndarray, np.ndarray]:
    sym3 = to_tok_head_chan(symbols, shape, axes)
    specs = np.asarray(specs, dtype=np.int64).reshape(-1, 6)
    bits = np.broadcast_to(np.asarray(bits, dtype=np.int64), (specs.shape[0],))
    parts = [bits_pack(chunk_symbols(sym3, s), int(b)) for s, b in zip(specs, bits)]
    offsets = np.concatenate([[0], np.cumsum([p.size for p in parts])]).astype(np.int64)
    flat = np.concatenate(parts) if parts else np.zeros(0, np.uint8)
    return flat.astype(np.uint8), offsets


def reference_unpack(flat, offsets, specs, bits, shape, axes) -> np.ndarray:
    out = np.zeros(int(np.prod(shape)), dtype=np.uint8)
    sym3 = to_tok_head_chan(out, shape, axes)  # a writable view into out
    specs = np.asarray(specs, dtype=np.int64).reshape(-1, 6)
    bits = np.broadcast_to(np.asarray(bits, dtype=np.int64), (specs.shape[0],))
    for k, (s, b) in enumerate(zip(specs, bits)):
        hs, he, cs, ce, ts, te = (int(x) for x in s)
        n = (he - hs) * (ce - cs) * (te - ts)
        vals = bits_unpack(flat[offsets[k]:offsets[k + 1]], int(b), n)
        sym3[ts:te, hs:he, cs:ce] = vals.reshape(he - hs, ce - cs, te - ts).transpose(2, 0, 1)
    return out


def random_specs(rng, T, H, C, n_max=6, full_tokens=False, partition=False):
    """Random chunk boxes.  partition=True: boxes tile the (h, c, t) space."""
    if partition:
        specs = []
        for h in range(H):
            c = 0
            while c < C:
                w = int(rng.integers(1, C - c + 1))
                if full_tokens:
                    specs.append([h, h + 1, c, c + w, 0, T])
                else:
                    t = 0
                    while t < T:
                        l = int(rng.integers(1, T - t + 1))
                        specs.append([h, h + 1, c, c + w, t, t + l])
                        t += l
                c += w
        return np.asarray(specs, dtype=np.int64)
    specs = []
    for _ in range(int(rng.integers(1, n_max + 1))):
        hs = int(rng.integers(0, H)); he = int(rng.integers(hs + 1, H + 1))
        cs = int(rng.integers(0, C)); ce = int(rng.integers(cs + 1, C + 1))
        if full_tokens:
            ts, te = 0, T
        else:
            ts = int(rng.integers(0, T)); te = int(rng.integers(ts + 1, T + 1))
        specs.append([hs, he, cs, ce, ts, te])
    return np.asarray(specs, dtype=np.int64)

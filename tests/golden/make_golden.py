"""Writes the golden fixtures in this folder.

The vectors come from the format's definition (tests/bitref.py: numpy bit
lists, LSB-first, head/channel/token order by fancy indexing), not from the
oracle or the HIP library, so both can be checked against them.  Re-running
the script reproduces the files bit for bit (fixed seeds).

  python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
from tests import bitref  # noqa: E402

CASES = []


def add(name, symbols, shape, axes, specs, bits):
    specs = np.asarray(specs, np.int64).reshape(-1, 6)
    bits_arr = np.broadcast_to(np.asarray(bits, np.int64), (specs.shape[0],)).copy()
    flat, offsets = bitref.reference_stream(symbols, shape, axes, specs, bits_arr)
    unpacked = bitref.reference_unpack(flat, offsets, specs, bits_arr, shape, axes)
    CASES.append(name)
    np.savez(HERE / f"{name}.npz", symbols=np.asarray(symbols, np.uint8).reshape(-1),
             shape=np.asarray(shape, np.int64), axes=np.asarray(axes, np.int64), specs=specs,
             bits=bits_arr, stream=flat, offsets=offsets, unpacked=unpacked)


def main():
    rng = np.random.default_rng(20260101)
    # 1. linear [1, 1, 37] streams, every bit width
    vals = rng.integers(0, 256, 37, dtype=np.uint8)
    for b in range(1, 9):
        add(f"linear_b{b}", vals, [1, 1, 37], [0, 1, 2, -1], [[0, 1, 0, 37, 0, 1]], b)
    # 2. token/head/head_dim layer view, planner-like channel chunks, bits 8 and 3
    T, H, C = 24, 2, 32
    sym = rng.integers(0, 256, T * H * C, dtype=np.uint8)
    specs = [[h, h + 1, c, c + 16, 0, T] for h in range(H) for c in (0, 16)]
    add("kv_view_b8", sym, [T, H, C], [0, 1, 2, -1], specs, 8)
    add("kv_view_b3", sym, [T, H, C], [0, 1, 2, -1], specs, 3)
    # 3. rank-4 layout with a layer axis, token-split boxes, mixed bit widths
    T, H, C = 9, 3, 5
    sym = rng.integers(0, 256, T * H * C, dtype=np.uint8)
    specs = [[0, 2, 0, 5, 0, 4], [0, 2, 0, 5, 4, 9], [2, 3, 0, 2, 0, 9], [2, 3, 2, 5, 0, 9]]
    add("rank4_mixed", sym, [H, 1, T, C], [2, 0, 3, 1], specs, [8, 5, 2, 7])
    # 4. partially covered tensor: the rest unpacks to zero
    T, H, C = 7, 2, 6
    sym = rng.integers(0, 256, T * H * C, dtype=np.uint8)
    add("partial_b4", sym, [T, H, C], [0, 1, 2, -1], [[1, 2, 1, 5, 2, 6]], 4)
    # 5. paged scatter of a [2, T, H, C] byte view into a kv-first cache
    T, H, C, bs, NB = 21, 2, 8, 4, 9
    value = rng.integers(0, 256, (2, T, H, C), dtype=np.uint8)
    ids = np.array([7, 2, 5, 0, 8, 3], np.int64)
    cache = rng.integers(0, 256, (2, NB, bs, H, C), dtype=np.uint8)
    expect = cache.copy()
    padded = np.zeros((2, ids.size * bs, H, C), np.uint8)
    padded[:, :T] = value
    expect[:, ids] = padded.reshape(2, ids.size, bs, H, C)
    np.savez(HERE / "scatter_kv_first.npz", value=value, ids=ids, cache=cache, expect=expect,
             tokens=np.int64(T))
    (HERE / "CASES.txt").write_text("\n".join(CASES + ["scatter_kv_first"]) + "\n")


if __name__ == "__main__":
    main()

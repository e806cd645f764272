"""Pins the CPU oracle (oracle/layout_oracle.c) to independent statements of
the reference's format, so that a plausible mistake in the oracle (wrong bit
order, shift, index or chunk order, a dropped zero-fill) fails here.

Independent statements used:
  * the bit-list definition in tests/bitref.py (numpy packbits/unpackbits,
    LSB-first) and numpy fancy indexing for the head/channel/token order;
  * for b = 8, the closed form "stream = S[ts:te, hs:he, cs:ce] transposed to
    head, channel, token" (identity packing, bitpack_layout_cuda.cu:74-76);
  * the KIVI adapter's own 2- and 4-bit packers (kivi_adapter.py:34-54):
    byte = s0 | s1 << 4 and byte = s0 | s1 << 2 | s2 << 4 | s3 << 6;
  * the pure linear [1, 1, N] single-chunk packing of cachegen_adapter.py:117-142;
  * numpy fancy-index assignment for the paged scatter (index_copy_ along the
    block axis, benchmark_utils.py:434-444) and the paged gather.
"""
import numpy as np
import pytest

from oracle import oracle
from tests import bitref

RNG = np.random.default_rng(1234)


@pytest.mark.parametrize("bits", range(1, 9))
def test_unpack_symbol_matches_bit_list(bits):
    rng = np.random.default_rng(bits)
    n = 97
    vals = rng.integers(0, 1 << bits, n, dtype=np.uint8)
    stream = bitref.bits_pack(vals, bits)
    got = [oracle.unpack_symbol(stream, i, bits) for i in range(n)]
    assert np.array_equal(np.array(got, np.uint8), vals)


def test_unpack_symbol_window_past_end_reads_zero():
    # bits 7, symbol 1 spans bytes 0..1; with a 1-byte buffer the high byte of
    # the 16-bit window is past the chunk and must read as 0 (cu:82-87).
    assert oracle.unpack_symbol(np.array([0xFF], np.uint8), 1, 7) == 0x01
    assert oracle.unpack_symbol(np.array([0xFF, 0xFF], np.uint8), 1, 7) == 0x7F


@pytest.mark.parametrize("bits", [2, 4])
def test_linear_pack_matches_kivi_packers(bits):
    rng = np.random.default_rng(7)
    n = 1000
    vals = rng.integers(0, 1 << bits, n, dtype=np.uint8)
    flat, offs = oracle.pack_canonical(vals, bits, [[0, 1, 0, n, 0, 1]], [1, 1, n], [0, 1, 2, -1])
    if bits == 4:
        pairs = vals.reshape(-1, 2)
        kivi = (pairs[:, 0] | (pairs[:, 1] << 4)).astype(np.uint8)
    else:
        g = vals.reshape(-1, 4)
        kivi = (g[:, 0] | (g[:, 1] << 2) | (g[:, 2] << 4) | (g[:, 3] << 6)).astype(np.uint8)
    assert offs.tolist() == [0, n * bits // 8]
    assert np.array_equal(flat, kivi)


def test_bits8_is_plane_major_transpose():
    T, H, C = 37, 3, 10
    sym = RNG.integers(0, 256, (T, H, C), dtype=np.uint8)
    specs = [[0, 2, 0, 10, 0, 37], [2, 3, 0, 4, 0, 37], [2, 3, 4, 10, 5, 37], [2, 3, 4, 10, 0, 5]]
    flat, offs = oracle.pack_canonical(sym, 8, specs, [T, H, C], [0, 1, 2, -1])
    expect = np.concatenate([sym[s[4]:s[5], s[0]:s[1], s[2]:s[3]].transpose(1, 2, 0).ravel()
                             for s in specs])
    assert np.array_equal(flat, expect)
    out = oracle.unpack_canonical(flat, offs, 8, specs, [T, H, C], [0, 1, 2, -1])
    assert np.array_equal(out.reshape(T, H, C), sym)


LAYOUTS = [
    (["token", "head", "head_dim"], [0, 1, 2, -1]),
    (["head", "token", "head_dim"], [1, 0, 2, -1]),
    (["head", "head_dim", "token"], [2, 0, 1, -1]),
    (["layer", "token", "head", "head_dim"], [1, 2, 3, 0]),
    (["token", "layer", "head_dim", "head"], [0, 3, 2, 1]),
]


def _shape_for(layout, T, H, C):
    size = {"token": T, "head": H, "head_dim": C, "layer": 1}
    return [size[a] for a in layout]


@pytest.mark.parametrize("bits", range(1, 9))
@pytest.mark.parametrize("li", range(len(LAYOUTS)))
def test_pack_and_unpack_match_bit_list_brute_force(bits, li):
    layout, axes = LAYOUTS[li]
    rng = np.random.default_rng(100 * bits + li)
    for trial in range(6):
        T, H, C = (int(x) for x in rng.integers(1, [8, 4, 6]))
        shape = _shape_for(layout, T, H, C)
        sym = rng.integers(0, 256, int(np.prod(shape)), dtype=np.uint8)
        specs = bitref.random_specs(rng, T, H, C, partition=bool(trial % 2))
        # the pack masks symbols to b bits; compare against masked inputs
        flat, offs = oracle.pack_canonical(sym, bits, specs, shape, axes)
        ref_flat, ref_offs = bitref.reference_stream(sym, shape, axes, specs, bits)
        assert np.array_equal(offs, ref_offs)
        assert np.array_equal(flat, ref_flat)
        out = oracle.unpack_canonical(flat, offs, bits, specs, shape, axes)
        ref_out = bitref.reference_unpack(flat, offs, specs, bits, shape, axes)
        if trial % 2:  # partition: overlaps impossible, unique answer
            assert np.array_equal(out, ref_out)
            assert np.array_equal(out, sym & ((1 << bits) - 1))


def test_unpack_leaves_uncovered_bytes_zero():
    T, H, C = 9, 2, 5
    specs = [[1, 2, 1, 4, 2, 7]]
    vals = RNG.integers(1, 256, 3 * 5, dtype=np.uint8)
    flat = bitref.bits_pack(vals, 8)
    out = oracle.unpack_canonical(flat, [0, flat.size], 8, specs, [T, H, C], [0, 1, 2, -1])
    out3 = out.reshape(T, H, C)
    mask = np.zeros((T, H, C), bool)
    mask[2:7, 1, 1:4] = True
    assert np.all(out3[~mask] == 0)
    assert np.array_equal(out3[2:7, 1, 1:4].transpose(1, 0).ravel(), vals)


@pytest.mark.parametrize("bits", range(1, 9))
def test_pack_of_unpack_is_identity_on_canonical_streams(bits):
    rng = np.random.default_rng(bits + 50)
    T, H, C = 11, 3, 7
    specs = bitref.random_specs(rng, T, H, C, partition=True)
    offs = oracle.chunk_offsets(specs, bits)
    # canonical stream: random symbols, zero pad bits
    parts = []
    for k, s in enumerate(specs):
        n = int((s[1] - s[0]) * (s[3] - s[2]) * (s[5] - s[4]))
        parts.append(bitref.bits_pack(rng.integers(0, 1 << bits, n, dtype=np.uint8), bits))
    flat = np.concatenate(parts)
    sym = oracle.unpack_canonical(flat, offs, bits, specs, [T, H, C], [0, 1, 2, -1])
    again, offs2 = oracle.pack_canonical(sym, bits, specs, [T, H, C], [0, 1, 2, -1])
    assert np.array_equal(offs, offs2)
    assert np.array_equal(again, flat)


def test_checks_catch_planted_mistakes():
    """The brute force is not vacuous: MSB-first bit order or a channel-fastest
    chunk order would be told apart from the reference format."""
    vals = np.array([1, 2, 3, 0, 1], np.uint8)
    lsb = bitref.bits_pack(vals, 3)
    mat = np.unpackbits(vals[:, None], axis=1, bitorder="little")[:, :3][:, ::-1]
    msb = np.packbits(mat.reshape(-1), bitorder="little")
    assert not np.array_equal(lsb, msb)
    sym = np.arange(2 * 1 * 3, dtype=np.uint8).reshape(2, 1, 3)
    tok_fast = bitref.chunk_symbols(sym, [0, 1, 0, 3, 0, 2])
    chan_fast = sym[:, 0, :].reshape(-1)
    assert not np.array_equal(tok_fast, chan_fast)
    flat, _ = oracle.pack_canonical(sym, 8, [[0, 1, 0, 3, 0, 2]], [2, 1, 3], [0, 1, 2, -1])
    assert np.array_equal(flat, tok_fast)


@pytest.mark.parametrize("blocks_first", [False, True])
def test_scatter_matches_fancy_index_assignment(blocks_first):
    rng = np.random.default_rng(3)
    NB, bs, H, C, T = 12, 4, 2, 6, 17
    nblk = -(-T // bs)
    ids = rng.permutation(NB)[:nblk]
    value = rng.integers(0, 256, (2, T, H, C), dtype=np.uint8)
    shape = (NB, 2, bs, H, C) if blocks_first else (2, NB, bs, H, C)
    cache = rng.integers(0, 256, shape, dtype=np.uint8)
    expect = cache.copy()
    padded = np.zeros((2, nblk * bs, H, C), np.uint8)
    padded[:, :T] = value
    blocks = padded.reshape(2, nblk, bs, H, C)
    if blocks_first:
        expect[ids] = blocks.transpose(1, 0, 2, 3, 4)
    else:
        expect[:, ids] = blocks
    oracle.scatter_kv_cache(value, T, H, C, ids, cache, blocks_first)
    assert np.array_equal(cache, expect)
    back = oracle.gather_kv_cache(cache, ids, blocks_first).reshape(2, nblk * bs, H, C)
    assert np.array_equal(back, padded)


def test_scatter_rejects_bad_block_ids():
    cache = np.zeros((2, 4, 2, 1, 4), np.uint8)
    with pytest.raises(RuntimeError, match="block id out of range"):
        oracle.scatter_kv_cache(np.zeros(2 * 2 * 4, np.uint8), 2, 1, 4, [4], cache)


@pytest.mark.parametrize("specs,bits,offsets,msg", [
    ([[0, 1, 0, 4, 0, 4]], [9], [0, 16], "1..8 bit"),
    ([[0, 1, 0, 4, 0, 4]], [8], [0, 15], "byte size mismatch"),
    ([[0, 3, 0, 4, 0, 4]], [8], [0, 48], "head range"),
    ([[0, 1, 2, 2, 0, 4]], [8], [0, 0], "channel range"),
    ([[0, 1, 0, 4, 0, 5]], [8], [0, 20], "token range"),
])
def test_oracle_validation_messages(specs, bits, offsets, msg):
    with pytest.raises(RuntimeError, match=msg):
        oracle.unpack_canonical(np.zeros(64, np.uint8), offsets, bits, specs, [4, 2, 4],
                                [0, 1, 2, -1])

"""Pins the dequant oracle (oracle/dequant_oracle.c) to independent
statements, so that a plausible mistake in it (a swapped K/V stream or bit
width, a wrong centre, a dropped rounding case, a transposed KIVI order, a
fused vs unfused multiply-add) fails here.

Independent statements used:
  * numpy float16 casts (every half pattern; rounding edge cases) and torch
    bfloat16 casts, both round to nearest even;
  * the reference's unfused Python paths restated with torch/numpy ops in
    tests/dqref.py (linear unpack, `(q - c) / c * max`, KIVI's packers and
    orders, block-by-block assignment);
  * closed forms: CacheGen symbols 0, c and 2c dequantize to exactly -max, 0
    and +max; KIVI body values with scale 1 and zero 0 are the symbols.
"""
import numpy as np
import pytest
import torch

from oracle import oracle
from tests import bitref, dqref


# ---------------------------------------------------------------------------
# Conversions
# ---------------------------------------------------------------------------

def test_half_to_float_every_pattern():
    pats = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ref = pats.view(np.float16).astype(np.float32)
    got = np.array([oracle.half_to_float(int(h)) for h in pats], dtype=np.float32)
    finite = ~np.isnan(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[~finite]))


def _half_edge_floats() -> np.ndarray:
    halves = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (halves[:-1] + halves[1:]) / 2          # exact ties between neighbours
    vals = [halves, mids, np.nextafter(mids, 0), np.nextafter(mids, np.inf),
            np.array([65504.0, 65519.996, 65520.0, 1e6, 2.0 ** -25, 2.0 ** -24, 2.0 ** -26,
                      np.nextafter(2.0 ** -25, 1), 0.0])]
    v = np.concatenate(vals).astype(np.float32)
    return np.concatenate([v, -v])


def test_float_to_half_round_to_nearest_even():
    rng = np.random.default_rng(7)
    rand = (rng.standard_normal(20000) * np.exp2(rng.integers(-30, 20, 20000))).astype(np.float32)
    vals = np.concatenate([_half_edge_floats()[::7], rand, np.array([np.inf, -np.inf], np.float32)])
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.float_to_half(float(x)) for x in vals], dtype=np.uint16)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, [(float(vals[i]), hex(got[i]), hex(ref[i])) for i in bad[:5]]


def test_float_to_bf16_round_to_nearest_even():
    rng = np.random.default_rng(8)
    base = rng.integers(0, 0x7F7F, 4000, dtype=np.uint32) << 16
    ties = base | 0x8000                                  # exactly halfway
    vals_u = np.concatenate([base, ties, ties + 1, ties - 1, base | 0x7FFF,
                             np.array([0x7F7FFFFF, 0x7F7F8000, 0x00008000, 0x00018000],
                                      np.uint32)])
    vals_u = np.concatenate([vals_u, vals_u | 0x80000000]).astype(np.uint32)
    vals = vals_u.view(np.float32)
    ref = torch.from_numpy(vals.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([oracle.float_to_bf16(float(x)) for x in vals], dtype=np.uint16)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, [(hex(vals_u[i]), hex(got[i]), hex(ref[i])) for i in bad[:5]]


# ---------------------------------------------------------------------------
# CacheGen
# ---------------------------------------------------------------------------

def _cache_bits(cache: torch.Tensor) -> np.ndarray:
    return cache.view(torch.int16).numpy().view(np.uint16)


def _make_cachegen(rng, tokens, heads, head_dim, key_bits, value_bits, max_dtype, gap=3):
    C = heads * head_dim
    kq = rng.integers(0, 1 << key_bits, tokens * C, dtype=np.uint8)
    vq = rng.integers(0, 1 << value_bits, tokens * C, dtype=np.uint8)
    ks, vs = bitref.bits_pack(kq, key_bits), bitref.bits_pack(vq, value_bits)
    stream = np.concatenate([np.full(gap, 0xAB, np.uint8), ks, np.full(gap, 0xCD, np.uint8), vs,
                             np.full(5, 0xEF, np.uint8)])
    koff, voff = gap, gap + ks.size + gap
    mk = (rng.random(tokens) * 4 + 0.01).astype(max_dtype)
    mv = (rng.random(tokens) * 4 + 0.01).astype(max_dtype)
    return stream, koff, ks.size, voff, vs.size, mk, mv


@pytest.mark.parametrize("blocks_first", [False, True])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("max_dtype", [np.float16, np.float32])
@pytest.mark.parametrize("key_bits,value_bits,key_bins,value_bins",
                         [(5, 4, 32, 16), (3, 2, 8, 4), (8, 6, 256, 40), (1, 7, 2, 100)])
def test_cachegen_cache_matches_unfused_reference(blocks_first, out_dtype, max_dtype, key_bits,
                                                  value_bits, key_bins, value_bins):
    rng = np.random.default_rng(key_bits * 10 + value_bits)
    tokens, heads, head_dim, bs, nb = 45, 3, 8, 8, 11
    stream, koff, kb, voff, vb, mk, mv = _make_cachegen(rng, tokens, heads, head_dim, key_bits,
                                                        value_bits, max_dtype)
    ids = [7, 2, -1, 9, 0, 11]                      # -1 and 11 (== NB) are skipped
    shape = (nb, 2, bs, heads, head_dim) if blocks_first else (2, nb, bs, heads, head_dim)
    init = torch.from_numpy(rng.integers(0, 1 << 15, int(np.prod(shape)), dtype=np.int16)
                            .reshape(shape)).view(out_dtype)
    ref = init.clone()
    dqref.cachegen_reference_cache(stream, koff, kb, voff, vb, key_bits, value_bits, key_bins,
                                   value_bins, mk, mv, ref, blocks_first, ids, tokens, heads,
                                   head_dim)
    got = _cache_bits(init.clone())
    oracle.cachegen_to_kv_cache(stream, koff, kb, voff, vb, key_bits, value_bits, key_bins,
                                value_bins, mk, mv, got, out_dtype == torch.bfloat16,
                                blocks_first, ids, tokens, heads, head_dim)
    exp = _cache_bits(ref)
    # bins = 2 gives c = 0: quotients are NaN / inf.  NaN payloads are not
    # pinned (they differ between hosts); positions and all other bits are.
    nan_ref = np.isnan(ref.float().numpy())
    nan_got = np.isnan(torch.from_numpy(got.view(np.int16)).view(out_dtype).float().numpy())
    assert np.array_equal(nan_got, nan_ref)
    assert np.array_equal(got[~nan_ref], exp[~nan_ref])


def test_cachegen_closed_form_levels():
    """Symbols 0, c, 2c dequantize to exactly -max, 0, +max."""
    bins, bits = 32, 5
    c = bins // 2 - 1
    tokens, heads, head_dim = 16, 1, 8
    q = np.tile(np.array([0, c, 2 * c, 0, c, 2 * c, c, 0], np.uint8), tokens)
    s = bitref.bits_pack(q, bits)
    stream = np.concatenate([s, s])
    mk = np.linspace(0.5, 3.0, tokens).astype(np.float32)
    cache = np.zeros((2, 2, 8, heads, head_dim), np.uint16)
    oracle.cachegen_to_kv_cache(stream, 0, s.size, s.size, s.size, bits, bits, bins, bins, mk,
                                mk, cache, True, False, [0, 1], tokens, heads, head_dim)
    vals = torch.from_numpy(cache.view(np.int16)).view(torch.bfloat16).float().numpy()
    k = vals[0].reshape(tokens, 8)
    mx = torch.from_numpy(mk).to(torch.bfloat16).float().numpy()
    expect = np.stack([-mx, 0 * mx, mx, -mx, 0 * mx, mx, 0 * mx, -mx], axis=1)
    assert np.array_equal(k, expect)


def test_cachegen_short_stream_reads_zero():
    """Symbols past key_bytes decode as 0 (bitpack_layout_cuda.cu:305-311)."""
    bits, bins, tokens, heads, head_dim = 4, 16, 8, 1, 8
    q = np.full(tokens * 8, 9, np.uint8)
    s = bitref.bits_pack(q, bits)
    short = s.size // 2
    mk = np.ones(tokens, np.float32)
    cache = np.zeros((2, 1, 8, 1, 8), np.uint16)
    oracle.cachegen_to_kv_cache(np.concatenate([s, s]), 0, short, s.size, s.size, bits, bits, bins,
                                bins, mk, mk, cache, False, False, [0], tokens, heads, head_dim)
    k = cache[0].reshape(-1).view(np.float16).astype(np.float32)
    c = bins // 2 - 1
    assert np.all(k[: short * 2] == np.float32((9 - c) / c).astype(np.float16))
    assert np.all(k[short * 2:] == -1.0)


def test_cachegen_dense_matches_unfused_reference():
    rng = np.random.default_rng(3)
    layers, tokens, heads, head_dim = 3, 21, 2, 12
    C = heads * head_dim
    bits = [5, 3, 8, 4, 2, 6]
    kbins, vbins = [32, 8, 200], [16, 4, 64]
    segs = [bitref.bits_pack(rng.integers(0, 1 << b, tokens * C, dtype=np.uint8), b) for b in bits]
    segs[4] = segs[4][:-3]                          # a short segment reads zeros at its end
    offs = np.concatenate([[0], np.cumsum([s.size for s in segs])]).astype(np.int64)
    stream = np.concatenate(segs)
    mk = (rng.random(layers * tokens) * 2 + 0.1).astype(np.float16)
    mv = (rng.random(layers * tokens) * 2 + 0.1).astype(np.float16)
    ref = dqref.cachegen_reference_dense(stream, offs, bits, kbins, vbins, mk, mv, tokens, heads,
                                         head_dim)
    got = oracle.cachegen_unpack_dequantize(stream, offs, bits, kbins, vbins, mk, mv, tokens,
                                            heads, head_dim)
    assert np.array_equal(got.view(np.uint16), ref.numpy().view(np.uint16))


def test_cachegen_oracle_rejects_bad_ranges():
    cache = np.zeros((2, 1, 4, 1, 8), np.uint16)
    m = np.ones(4, np.float32)
    with pytest.raises(RuntimeError, match="exceed"):
        oracle.cachegen_to_kv_cache(np.zeros(10, np.uint8), 0, 8, 4, 8, 4, 4, 16, 16, m, m, cache,
                                    False, False, [0], 4, 1, 8)
    with pytest.raises(RuntimeError, match="bins"):
        oracle.cachegen_to_kv_cache(np.zeros(32, np.uint8), 0, 16, 16, 16, 4, 4, 1, 16, m, m,
                                    cache, False, False, [0], 4, 1, 8)


# ---------------------------------------------------------------------------
# KIVI
# ---------------------------------------------------------------------------

def _make_kivi(rng, tokens, sink, heads, head_dim, bits, group, meta_dtype, kivi_container):
    C = heads * head_dim
    body = tokens - sink
    kq = rng.integers(0, 1 << bits, body * C, dtype=np.uint8).reshape(body, C)
    vq = rng.integers(0, 1 << bits, body * C, dtype=np.uint8).reshape(body, C)
    korder = dqref.kivi_key_order(kq, heads, head_dim)
    vorder = dqref.kivi_value_order(vq, heads, head_dim)
    if kivi_container:
        ks, vs = dqref.kivi_pack(korder, bits), dqref.kivi_pack(vorder, bits)
    else:
        ks, vs = bitref.bits_pack(korder, bits), bitref.bits_pack(vorder, bits)
    stream = np.concatenate([ks, np.zeros(1, np.uint8), vs])
    kg = (body + group - 1) // group
    vg = (C + group - 1) // group
    meta = dict(
        key_scale=(rng.random(kg * C) * 0.5 + 0.01).astype(meta_dtype),
        key_zero=(rng.standard_normal(kg * C)).astype(meta_dtype),
        value_scale=(rng.random(body * vg) * 0.5 + 0.01).astype(meta_dtype),
        value_zero=(rng.standard_normal(body * vg)).astype(meta_dtype),
        key_sink=(rng.standard_normal(sink * C)).astype(meta_dtype),
        value_sink=(rng.standard_normal(sink * C)).astype(meta_dtype),
    )
    return stream, 0, ks.size, ks.size + 1, vs.size, meta


@pytest.mark.parametrize("bits,nibble3", [(2, False), (3, True), (3, False), (4, False),
                                          (8, False), (5, False)])
@pytest.mark.parametrize("blocks_first", [False, True])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("meta_dtype", [np.float16, np.float32])
def test_kivi_cache_matches_reference(bits, nibble3, blocks_first, out_dtype, meta_dtype):
    rng = np.random.default_rng(bits * 7 + nibble3)
    tokens, sink, heads, head_dim, bs, nb, group = 40, 6, 2, 8, 8, 9, 5
    stream, koff, kb, voff, vb, meta = _make_kivi(rng, tokens, sink, heads, head_dim, bits, group,
                                                  meta_dtype, nibble3 or bits in (2, 4, 8))
    ids = [4, 8, 1, -3, 6]
    shape = (nb, 2, bs, heads, head_dim) if blocks_first else (2, nb, bs, heads, head_dim)
    init = torch.from_numpy(rng.integers(0, 1 << 14, int(np.prod(shape)), dtype=np.int16)
                            .reshape(shape)).view(out_dtype)
    ref = init.clone()
    dqref.kivi_reference_cache(stream, koff, kb, voff, vb, bits, nibble3, group, sink,
                               meta["key_scale"], meta["key_zero"], meta["value_scale"],
                               meta["value_zero"], meta["key_sink"], meta["value_sink"], ref,
                               blocks_first, ids, tokens, heads, head_dim)
    got = _cache_bits(init.clone())
    oracle.kivi_to_kv_cache(stream, koff, kb, voff, vb, bits, nibble3, group, sink,
                            meta["key_scale"], meta["key_zero"], meta["value_scale"],
                            meta["value_zero"], meta["key_sink"], meta["value_sink"], got,
                            out_dtype == torch.bfloat16, blocks_first, ids, tokens, heads,
                            head_dim)
    assert np.array_equal(got, _cache_bits(ref))


def test_kivi_identity_scale_returns_symbols():
    """scale 1, zero 0: body values equal the symbols (order check)."""
    rng = np.random.default_rng(11)
    tokens, sink, heads, head_dim, bits, group = 16, 0, 2, 4, 4, 4
    C = heads * head_dim
    kq = rng.integers(0, 16, tokens * C, dtype=np.uint8).reshape(tokens, C)
    vq = rng.integers(0, 16, tokens * C, dtype=np.uint8).reshape(tokens, C)
    ks = dqref.kivi_pack(dqref.kivi_key_order(kq, heads, head_dim), bits)
    vs = dqref.kivi_pack(dqref.kivi_value_order(vq, heads, head_dim), bits)
    stream = np.concatenate([ks, vs])
    one = np.ones(max(tokens * C, 64), np.float32)
    zero = np.zeros_like(one)
    cache = np.zeros((2, 2, 8, heads, head_dim), np.uint16)
    oracle.kivi_to_kv_cache(stream, 0, ks.size, ks.size, vs.size, bits, False, group, sink, one,
                            zero, one, zero, zero[:0], zero[:0], cache, False, False, [0, 1],
                            tokens, heads, head_dim)
    k = cache[0].reshape(tokens, C).view(np.float16).astype(np.float32)
    v = cache[1].reshape(tokens, C).view(np.float16).astype(np.float32)
    assert np.array_equal(k, kq.astype(np.float32))
    assert np.array_equal(v, vq.astype(np.float32))


def test_kivi_multiply_add_is_fused():
    """A case where fmaf(s, scale, zero) and round(round(s * scale) + zero)
    differ: the oracle must give the fused result."""
    s, scale = 3, np.float32(1 + 2 ** -23)
    zero = np.float32(-3.0)
    fused = dqref.exact_fma32(np.array([s], np.float32), np.array([scale]), np.array([zero]))[0]
    unfused = np.float32(np.float32(s) * scale) + zero
    assert fused != unfused
    stream = dqref.kivi_pack(np.array([s, s], np.uint8), 2)
    one = np.array([scale], np.float32)
    z = np.array([zero], np.float32)
    cache = np.zeros((2, 1, 1, 1, 1), np.uint16)
    oracle.kivi_to_kv_cache(stream, 0, 1, 0, 1, 2, False, 1, 0, one, z, one, z, z[:0], z[:0],
                            cache, False, False, [0], 1, 1, 1)
    assert cache[0, 0, 0, 0, 0] == np.float32(fused).astype(np.float16).view(np.uint16)

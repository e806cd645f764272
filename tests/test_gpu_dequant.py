"""Parity of the HIP CacheGen and KIVI dequantize kernels
(liborigami_layout.so) with the CPU oracle (oracle/dequant_oracle.c).

Comparisons are bit-exact on the float16 / bfloat16 bits.  The one case with
bins = 2 (centre 0, so quotients are NaN or infinite) compares NaN positions
and every other bit.  Cases cover bits 1..8 for K and V independently, both
cache layouts, float16 / float32 maxima, float16 / bfloat16 caches, the
row kernel (C % 8 == 0) and the element kernel (C % 8 != 0 or an unaligned
cache), unaligned and short streams, skipped block ids, untouched tail
tokens, and one full Llama-3-8B layer (32768 tokens, 8 KV heads x 128).
KIVI cases cover bits 1..8 LSB-first and KIVI's 3-bit nibble container,
sink tokens, key/value groups, the row kernel and the element kernel, partial
token and channel tiles, blocks that split a lane's 16 tokens, and a full
Llama-3-8B layer.
"""
import numpy as np
import pytest
import torch

from oracle import oracle
from origami_amd.lossless import native_gpu
from tests import bitref, dqref

pytestmark = pytest.mark.gpu

BITS_CASES = [(5, 4, 32, 16), (3, 2, 8, 4), (8, 6, 256, 40), (1, 7, 4, 100), (4, 4, 16, 16),
              (2, 8, 4, 256), (6, 3, 64, 8), (7, 5, 128, 32)]


def _bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _make_case(rng, tokens, heads, head_dim, key_bits, value_bits, max_dtype, gap=3,
               short_key=0):
    C = heads * head_dim
    kq = rng.integers(0, 1 << key_bits, tokens * C, dtype=np.uint8)
    vq = rng.integers(0, 1 << value_bits, tokens * C, dtype=np.uint8)
    ks, vs = bitref.bits_pack(kq, key_bits), bitref.bits_pack(vq, value_bits)
    # the value stream ends exactly at the end of the bytestream allocation
    stream = np.concatenate([rng.integers(0, 256, gap, dtype=np.uint8), ks,
                             rng.integers(0, 256, gap, dtype=np.uint8), vs])
    koff, voff = gap, gap + ks.size + gap
    mk = (rng.random(tokens + 3) * 4 + 0.01).astype(max_dtype)
    mv = (rng.random(tokens + 3) * 4 + 0.01).astype(max_dtype)
    return stream, koff, ks.size - short_key, voff, vs.size, mk, mv


def _run_both(dev, rng, *, tokens, heads, head_dim, bs, nb, ids, key_bits, value_bits, key_bins,
              value_bins, out_dtype, max_dtype, blocks_first, gap=3, short_key=0,
              cache_offset=0):
    stream, koff, kb, voff, vb, mk, mv = _make_case(rng, tokens, heads, head_dim, key_bits,
                                                    value_bits, max_dtype, gap, short_key)
    shape = (nb, 2, bs, heads, head_dim) if blocks_first else (2, nb, bs, heads, head_dim)
    n = int(np.prod(shape))
    init = rng.integers(-(1 << 14), 1 << 14, n + cache_offset, dtype=np.int16)
    base = torch.from_numpy(init).to(dev).view(out_dtype)
    cache = base[cache_offset:].view(shape)
    expect = init[cache_offset:].view(np.uint16).reshape(shape).copy()
    oracle.cachegen_to_kv_cache(stream, koff, kb, voff, vb, key_bits, value_bits, key_bins,
                                value_bins, mk, mv, expect, out_dtype == torch.bfloat16,
                                blocks_first, ids, tokens, heads, head_dim)
    native_gpu.cachegen_unpack_dequantize_to_kv_cache(
        torch.from_numpy(stream).to(dev), key_offset=koff, key_bytes=kb, value_offset=voff,
        value_bytes=vb, key_bits=key_bits, value_bits=value_bits, key_bins=key_bins,
        value_bins=value_bins, max_key=torch.from_numpy(mk).to(dev),
        max_value=torch.from_numpy(mv).to(dev), kv_cache=cache,
        block_ids=torch.tensor(ids, dtype=torch.int64, device=dev), tokens=tokens, heads=heads,
        head_dim=head_dim)
    torch.cuda.synchronize(dev)
    return _bits16(cache), expect


@pytest.mark.parametrize("blocks_first", [False, True])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("max_dtype", [np.float16, np.float32])
@pytest.mark.parametrize("bc", range(len(BITS_CASES)))
def test_cachegen_cache_row_kernel(cuda_device, bc, max_dtype, out_dtype, blocks_first):
    kbits, vbits, kbins, vbins = BITS_CASES[bc]
    rng = np.random.default_rng(100 + bc)
    ids = [5, 12, 0, -1, 9, 3, 17, 7]           # -1 and 17 (== NB) are skipped
    got, exp = _run_both(cuda_device, rng, tokens=117, heads=4, head_dim=16, bs=16, nb=17,
                         ids=ids, key_bits=kbits, value_bits=vbits, key_bins=kbins,
                         value_bins=vbins, out_dtype=out_dtype, max_dtype=max_dtype,
                         blocks_first=blocks_first)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("case", ["c_not_multiple_of_8", "unaligned_cache", "wide_rows",
                                  "short_key_stream", "aligned_streams", "single_token"])
@pytest.mark.parametrize("blocks_first", [False, True])
def test_cachegen_cache_shapes(cuda_device, case, blocks_first):
    rng = np.random.default_rng(sum(map(ord, case)))
    kw = dict(tokens=70, heads=3, head_dim=16, bs=8, nb=12, ids=[3, 11, 0, 6, 8, 1, 2, 9, 10],
              key_bits=5, value_bits=3, key_bins=32, value_bins=8, out_dtype=torch.bfloat16,
              max_dtype=np.float16, blocks_first=blocks_first)
    if case == "c_not_multiple_of_8":
        kw.update(heads=3, head_dim=12)
    elif case == "unaligned_cache":
        kw.update(cache_offset=1)
    elif case == "wide_rows":                   # C = 4096: more groups per row than threads
        kw.update(heads=32, head_dim=128, tokens=37, bs=16, ids=[4, 0, 7], nb=8)
    elif case == "short_key_stream":            # symbols past key_bytes read 0
        kw.update(short_key=17)
    elif case == "aligned_streams":
        kw.update(gap=16)
    elif case == "single_token":
        kw.update(tokens=1, ids=[5])
    got, exp = _run_both(cuda_device, rng, **kw)
    assert np.array_equal(got, exp)


def test_cachegen_cache_zero_centre_nan_positions(cuda_device):
    """bins = 2 gives c = 0 ((s - 0) / 0 is NaN or inf), as in the reference."""
    rng = np.random.default_rng(5)
    # nb = 3: with two blocks the shape [2, 2, ...] would read as [NB, 2, ...]
    # (the reference's rule checks size(1) == 2 first, cpp:529)
    got, exp = _run_both(cuda_device, rng, tokens=32, heads=2, head_dim=8, bs=16, nb=3,
                         ids=[2, 0], key_bits=1, value_bits=2, key_bins=2, value_bins=3,
                         out_dtype=torch.float16, max_dtype=np.float32, blocks_first=False)
    g = got.view(np.float16)
    e = exp.view(np.float16)
    bad = np.nonzero((np.isnan(g) != np.isnan(e)) | (~np.isnan(e) & (got != exp)))
    assert bad[0].size == 0, [(tuple(int(x) for x in i), hex(got[i]), hex(exp[i]))
                              for i in list(zip(*bad))[:8]]


def test_cachegen_cache_llama3_8b_layer(cuda_device):
    """One full layer at the Llama-3-8B geometry (32768 tokens, 8 x 128,
    block size 16, permuted block table), 5-bit keys and 4-bit values."""
    rng = np.random.default_rng(8)
    tokens, bs = 32768, 16
    nb = tokens // bs + 64
    ids = rng.permutation(nb)[: tokens // bs]
    got, exp = _run_both(cuda_device, rng, tokens=tokens, heads=8, head_dim=128, bs=bs, nb=nb,
                         ids=ids.tolist(), key_bits=5, value_bits=4, key_bins=32, value_bins=16,
                         out_dtype=torch.bfloat16, max_dtype=np.float16, blocks_first=False,
                         gap=0)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("head_dim", [16, 12])
@pytest.mark.parametrize("max_dtype", [np.float16, np.float32])
def test_cachegen_dense_matches_oracle(cuda_device, head_dim, max_dtype):
    rng = np.random.default_rng(head_dim)
    layers, tokens, heads = 3, 45, 3
    C = heads * head_dim
    bits = [5, 3, 8, 4, 2, 6]
    kbins, vbins = [32, 8, 200], [16, 4, 64]
    segs = [bitref.bits_pack(rng.integers(0, 1 << b, tokens * C, dtype=np.uint8), b)
            for b in bits]
    segs[4] = segs[4][:-5]                       # short segment: trailing symbols read 0
    offs = np.concatenate([[1], 1 + np.cumsum([s.size for s in segs])]).astype(np.int64)
    stream = np.concatenate([np.zeros(1, np.uint8)] + segs)
    mk = (rng.random(layers * tokens) * 2 + 0.1).astype(max_dtype)
    mv = (rng.random(layers * tokens) * 2 + 0.1).astype(max_dtype)
    exp = oracle.cachegen_unpack_dequantize(stream, offs, bits, kbins, vbins, mk, mv, tokens,
                                            heads, head_dim)
    dev = cuda_device
    got = native_gpu.cachegen_unpack_dequantize(
        torch.from_numpy(stream).to(dev), torch.from_numpy(offs), torch.tensor(bits),
        torch.tensor(kbins), torch.tensor(vbins), torch.from_numpy(mk).to(dev),
        torch.from_numpy(mv).to(dev), tokens=tokens, heads=heads, head_dim=head_dim)
    assert got.shape == (layers, 2, heads, tokens, head_dim) and got.dtype == torch.float16
    assert np.array_equal(_bits16(got), exp.view(np.uint16))


def test_cachegen_extension_surface(cuda_device):
    """The reference's positional signatures (bitpack_layout_cuda.cpp:402-412,
    475-491) reach the same kernels."""
    ext = native_gpu.load_bitpack_cuda_extension()
    rng = np.random.default_rng(21)
    dev = cuda_device
    tokens, heads, head_dim, bs, nb = 32, 2, 8, 16, 4
    stream, koff, kb, voff, vb, mk, mv = _make_case(rng, tokens, heads, head_dim, 4, 4,
                                                    np.float16, gap=0)
    cache = torch.zeros((nb, 2, bs, heads, head_dim), dtype=torch.float16, device=dev)
    expect = np.zeros(cache.shape, np.uint16)
    oracle.cachegen_to_kv_cache(stream, koff, kb, voff, vb, 4, 4, 16, 16, mk, mv, expect, False,
                                True, [2, 0], tokens, heads, head_dim)
    ext.cachegen_unpack_dequantize_to_kv_cache_cuda(
        torch.from_numpy(stream).to(dev), koff, kb, voff, vb, 4, 4, 16, 16,
        torch.from_numpy(mk).to(dev), torch.from_numpy(mv).to(dev), cache,
        torch.tensor([2, 0], dtype=torch.int64, device=dev), tokens, heads, head_dim)
    assert np.array_equal(_bits16(cache), expect)
    out = ext.cachegen_unpack_dequantize_cuda(
        torch.from_numpy(stream).to(dev),
        torch.tensor([koff, koff + kb, voff + vb], dtype=torch.int64, device=dev),
        torch.tensor([4, 4], device=dev), torch.tensor([16], device=dev),
        torch.tensor([16], device=dev), torch.from_numpy(mk[:tokens]).to(dev),
        torch.from_numpy(mv[:tokens]).to(dev), tokens, heads, head_dim)
    assert out.shape == (1, 2, heads, tokens, head_dim)


def test_cachegen_errors(cuda_device):
    dev = cuda_device
    s = torch.zeros(64, dtype=torch.uint8, device=dev)
    m16 = torch.ones(8, dtype=torch.float16, device=dev)
    ids = torch.tensor([0], dtype=torch.int64, device=dev)
    kw = dict(key_offset=0, key_bytes=16, value_offset=16, value_bytes=16, key_bits=4,
              value_bits=4, key_bins=16, value_bins=16, max_key=m16, max_value=m16,
              block_ids=ids, tokens=8, heads=1, head_dim=4)
    cache = torch.zeros((2, 1, 8, 1, 4), dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="float16 or bfloat16"):
        native_gpu.cachegen_unpack_dequantize_to_kv_cache(s, **{**kw, "kv_cache": cache.float()})
    with pytest.raises(RuntimeError, match="supports only 1..8"):
        native_gpu.cachegen_unpack_dequantize_to_kv_cache(s, **{**kw, "kv_cache": cache,
                                                                "key_bits": 9})
    with pytest.raises(RuntimeError, match="bins must be greater than one"):
        native_gpu.cachegen_unpack_dequantize_to_kv_cache(s, **{**kw, "kv_cache": cache,
                                                                "value_bins": 1})
    with pytest.raises(RuntimeError, match="exceed bytestream length"):
        native_gpu.cachegen_unpack_dequantize_to_kv_cache(s, **{**kw, "kv_cache": cache,
                                                                "value_bytes": 60})
    with pytest.raises(RuntimeError, match="at least tokens values"):
        native_gpu.cachegen_unpack_dequantize_to_kv_cache(
            s, **{**kw, "kv_cache": cache, "max_key": m16[:4]})
    with pytest.raises(RuntimeError, match="tokens exceed destination block capacity"):
        native_gpu.cachegen_unpack_dequantize_to_kv_cache(s, **{**kw, "kv_cache": cache,
                                                                "tokens": 9,
                                                                "max_key": torch.ones(
                                                                    9, dtype=torch.float16,
                                                                    device=dev),
                                                                "max_value": torch.ones(
                                                                    9, dtype=torch.float16,
                                                                    device=dev)})
    with pytest.raises(RuntimeError, match="same dtype"):
        native_gpu.cachegen_unpack_dequantize_to_kv_cache(
            s, **{**kw, "kv_cache": cache, "max_value": m16.float()})
    with pytest.raises(RuntimeError, match="head shape mismatch"):
        native_gpu.cachegen_unpack_dequantize_to_kv_cache(s, **{**kw, "kv_cache": cache,
                                                                "head_dim": 8})


# ---------------------------------------------------------------------------
# KIVI
# ---------------------------------------------------------------------------

def _kivi_case(rng, tokens, sink, heads, head_dim, bits, nibble3, group, meta_dtype, gap=1,
               short_value=0):
    C = heads * head_dim
    body = tokens - sink
    kq = rng.integers(0, 1 << bits, body * C, dtype=np.uint8).reshape(body, C)
    vq = rng.integers(0, 1 << bits, body * C, dtype=np.uint8).reshape(body, C)
    korder = dqref.kivi_key_order(kq, heads, head_dim)
    vorder = dqref.kivi_value_order(vq, heads, head_dim)
    if nibble3:
        ks, vs = dqref.kivi_pack(korder, 3), dqref.kivi_pack(vorder, 3)
    else:
        ks, vs = bitref.bits_pack(korder, bits), bitref.bits_pack(vorder, bits)
    stream = np.concatenate([rng.integers(0, 256, gap, dtype=np.uint8), ks,
                             rng.integers(0, 256, gap, dtype=np.uint8), vs])
    kg = (body + group - 1) // group
    vg = (C + group - 1) // group
    meta = [(rng.random(kg * C) * 0.5 + 0.01).astype(meta_dtype),
            rng.standard_normal(kg * C).astype(meta_dtype),
            (rng.random(body * vg) * 0.5 + 0.01).astype(meta_dtype),
            rng.standard_normal(body * vg).astype(meta_dtype),
            rng.standard_normal(sink * C).astype(meta_dtype),
            rng.standard_normal(sink * C).astype(meta_dtype)]
    return stream, gap, ks.size, 2 * gap + ks.size, vs.size - short_value, meta


def _kivi_run_both(dev, rng, *, tokens, sink, heads, head_dim, bits, nibble3=False, group,
                   bs, nb, ids, out_dtype, meta_dtype, blocks_first, gap=1, short_value=0,
                   cache_offset=0):
    stream, koff, kb, voff, vb, meta = _kivi_case(rng, tokens, sink, heads, head_dim, bits,
                                                  nibble3, group, meta_dtype, gap, short_value)
    shape = (nb, 2, bs, heads, head_dim) if blocks_first else (2, nb, bs, heads, head_dim)
    n = int(np.prod(shape))
    init = rng.integers(-(1 << 14), 1 << 14, n + cache_offset, dtype=np.int16)
    cache = torch.from_numpy(init).to(dev).view(out_dtype)[cache_offset:].view(shape)
    expect = init[cache_offset:].view(np.uint16).reshape(shape).copy()
    oracle.kivi_to_kv_cache(stream, koff, kb, voff, vb, bits, nibble3, group, sink, *meta, expect,
                            out_dtype == torch.bfloat16, blocks_first, ids, tokens, heads,
                            head_dim)
    dm = [torch.from_numpy(m).to(dev) for m in meta]
    native_gpu.kivi_dequantize_to_kv_cache(
        torch.from_numpy(stream).to(dev), key_offset=koff, key_bytes=kb, value_offset=voff,
        value_bytes=vb, bits=bits, group_size=group, sink_tokens=sink, key_scale=dm[0],
        key_zero=dm[1], value_scale=dm[2], value_zero=dm[3], key_sink=dm[4], value_sink=dm[5],
        kv_cache=cache, block_ids=torch.tensor(ids, dtype=torch.int64, device=dev),
        tokens=tokens, heads=heads, head_dim=head_dim,
        symbol_packing="kivi" if nibble3 else "lsb")
    torch.cuda.synchronize(dev)
    return _bits16(cache), expect


KIVI_BITS = [(2, False), (3, True), (3, False), (4, False), (8, False), (1, False), (5, False),
             (6, False), (7, False)]


@pytest.mark.parametrize("blocks_first", [False, True])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("meta_dtype", [np.float16, np.float32])
@pytest.mark.parametrize("kb", range(len(KIVI_BITS)))
def test_kivi_row_kernel(cuda_device, kb, meta_dtype, out_dtype, blocks_first):
    bits, nibble3 = KIVI_BITS[kb]
    rng = np.random.default_rng(300 + kb)
    # body = 600 - 24 = 576 tokens: one full 512-token tile and a partial one;
    # C = 128: two channel tiles; group 32.
    ids = rng.permutation(45)[:38].tolist()
    ids[5] = -1
    got, exp = _kivi_run_both(cuda_device, rng, tokens=600, sink=24, heads=2, head_dim=64,
                              bits=bits, nibble3=nibble3, group=32, bs=16, nb=45, ids=ids,
                              out_dtype=out_dtype, meta_dtype=meta_dtype,
                              blocks_first=blocks_first)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("case", ["group16", "group64_sink128", "no_sink", "generic_group",
                                  "generic_head_dim", "unaligned_cache", "short_value_stream",
                                  "c_partial_tile", "block_size_7", "all_sink"])
def test_kivi_shapes(cuda_device, case):
    rng = np.random.default_rng(sum(map(ord, case)))
    kw = dict(tokens=300, sink=20, heads=4, head_dim=16, bits=2, group=32, bs=16, nb=40,
              ids=list(range(39, 20, -1)), out_dtype=torch.bfloat16, meta_dtype=np.float16,
              blocks_first=False)
    if case == "group16":
        kw.update(group=16)
    elif case == "group64_sink128":
        kw.update(tokens=1000, sink=128, group=64, ids=list(range(63)), nb=70)
    elif case == "no_sink":
        kw.update(sink=0)
    elif case == "generic_group":                # group % 16 != 0: element kernel
        kw.update(group=5, bits=3, nibble3=True)
    elif case == "generic_head_dim":             # head_dim % 8 != 0: element kernel
        kw.update(heads=3, head_dim=12, bits=4)
    elif case == "unaligned_cache":
        kw.update(cache_offset=1)
    elif case == "short_value_stream":           # symbols past value_bytes read 0
        kw.update(short_value=9)
    elif case == "c_partial_tile":               # C = 96: the second channel tile is partial
        kw.update(heads=3, head_dim=32, bits=4)
    elif case == "block_size_7":                 # lane tokens straddle blocks
        kw.update(bs=7, nb=50, ids=list(range(49, 6, -1)))
    elif case == "all_sink":
        kw.update(tokens=40, sink=40, ids=[3, 1, 2])
    got, exp = _kivi_run_both(cuda_device, rng, **kw)
    assert np.array_equal(got, exp)


def test_kivi_llama3_8b_layer(cuda_device):
    """A full layer at the Llama-3-8B geometry: 32768 tokens, 128 sink tokens,
    group 32, 2-bit KIVI, permuted block table."""
    rng = np.random.default_rng(9)
    tokens, bs = 32768, 16
    nb = tokens // bs + 32
    ids = rng.permutation(nb)[: tokens // bs].tolist()
    got, exp = _kivi_run_both(cuda_device, rng, tokens=tokens, sink=128, heads=8, head_dim=128,
                              bits=2, group=32, bs=bs, nb=nb, ids=ids, out_dtype=torch.bfloat16,
                              meta_dtype=np.float16, blocks_first=False, gap=0)
    assert np.array_equal(got, exp)


def test_kivi_extension_surface_and_errors(cuda_device):
    ext = native_gpu.load_bitpack_cuda_extension()
    dev = cuda_device
    rng = np.random.default_rng(4)
    tokens, sink, heads, head_dim, group = 64, 16, 2, 16, 16
    stream, koff, kb, voff, vb, meta = _kivi_case(rng, tokens, sink, heads, head_dim, 4, False,
                                                  group, np.float16)
    cache = torch.zeros((2, 5, 16, heads, head_dim), dtype=torch.float16, device=dev)
    expect = np.zeros(cache.shape, np.uint16)
    oracle.kivi_to_kv_cache(stream, koff, kb, voff, vb, 4, False, group, sink, *meta, expect,
                            False, False, [4, 0, 3, 1], tokens, heads, head_dim)
    dm = [torch.from_numpy(m).to(dev) for m in meta]
    ids = torch.tensor([4, 0, 3, 1], dtype=torch.int64, device=dev)
    s = torch.from_numpy(stream).to(dev)
    ext.kivi_dequantize_to_kv_cache_cuda(s, koff, kb, voff, vb, 4, group, sink, *dm, cache, ids,
                                         tokens, heads, head_dim)
    assert np.array_equal(_bits16(cache), expect)
    args = [s, koff, kb, voff, vb, 4, group, sink, *dm, cache, ids, tokens, heads, head_dim]
    bad = list(args)
    bad[6] = 0
    with pytest.raises(RuntimeError, match="group_size must be positive"):
        ext.kivi_dequantize_to_kv_cache_cuda(*bad)
    bad = list(args)
    bad[7] = tokens + 1
    with pytest.raises(RuntimeError, match="sink_tokens must be in"):
        ext.kivi_dequantize_to_kv_cache_cuda(*bad)
    bad = list(args)
    bad[8] = dm[0][:-1]
    with pytest.raises(RuntimeError, match="key metadata is too small"):
        ext.kivi_dequantize_to_kv_cache_cuda(*bad)
    bad = list(args)
    bad[10] = dm[2][:-1]
    with pytest.raises(RuntimeError, match="value metadata is too small"):
        ext.kivi_dequantize_to_kv_cache_cuda(*bad)
    bad = list(args)
    bad[13] = dm[5][:-1]
    with pytest.raises(RuntimeError, match="sink metadata is too small"):
        ext.kivi_dequantize_to_kv_cache_cuda(*bad)
    bad = list(args)
    bad[9] = dm[1].float()
    with pytest.raises(RuntimeError, match="same dtype"):
        ext.kivi_dequantize_to_kv_cache_cuda(*bad)
    bad = list(args)
    bad[5] = 9
    with pytest.raises(RuntimeError, match="supports only 1..8"):
        ext.kivi_dequantize_to_kv_cache_cuda(*bad)
    bad = list(args)
    bad[4] = len(stream)
    with pytest.raises(RuntimeError, match="exceed bytestream length"):
        ext.kivi_dequantize_to_kv_cache_cuda(*bad)

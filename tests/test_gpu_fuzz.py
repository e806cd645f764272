"""Seeded random restores and saves through the fused paged-cache entry points,
and seeded random CacheGen / KIVI dequantizing restores, each compared bit for
bit with the oracle.

Every case draws a token count (ragged or a multiple of 16), heads, head
bytes, symbol width, block size, cache layout, a permuted block table, a
misaligned stream pointer and a chunk plan.  The plan is either the planner's
(dense planes), the planner's boxes in reverse order (regular but not dense),
or full-token boxes of random channel widths.  The draws cross the row
kernels' addressing modes (aligned16, window, shift, bytes), workgroup sizes
and the stream-end fallback.
"""
import numpy as np
import pytest
import torch

from oracle import oracle
from origami_amd.layout import kv_symbol_layout
from origami_amd.lossless import native_gpu
from origami_amd.lossless.chunking import plan_head_channel_chunks
from tests import bitref

pytestmark = pytest.mark.gpu


def _plan(rng, kind, T2, H, C):
    if kind == "random":
        return bitref.random_specs(rng, T2, H, C, partition=True, full_tokens=True)
    target = int(rng.choice([64, 1024, 1 << 14, 1 << 16]))
    specs = np.asarray([[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
                         c.layout.channel_end, 0, T2]
                        for c in plan_head_channel_chunks(
                            layer_index=0, num_heads=H, head_dim=C, token_count=T2,
                            bytes_per_symbol=1, min_bytes=target, target_bytes=target,
                            max_bytes=target)], dtype=np.int64)
    return specs[::-1].copy() if kind == "reversed" else specs


@pytest.mark.parametrize("seed", range(40))
def test_random_restore_and_save(cuda_device, seed):
    rng = np.random.default_rng(1000 + seed)
    T = int(rng.integers(16, 3000)) if seed % 2 else 16 * int(rng.integers(1, 190))
    H = int(rng.choice([1, 2, 4, 8]))
    C = 16 * int(rng.integers(1, 17))
    bits = int(rng.integers(1, 9))
    bs = int(rng.choice([8, 16, 32]))
    blocks_first = bool(rng.integers(0, 2))
    shift = int(rng.choice([0, 0, 1, 2, 3, 4]))
    kind = ["planner", "reversed", "random"][seed % 3]
    specs = _plan(rng, kind, 2 * T, H, C)
    case = (T, H, C, bits, bs, blocks_first, shift, kind, len(specs))

    value = rng.integers(0, 256, (2, T, H, C), dtype=np.uint8)
    flat, offs = oracle.pack_canonical(value.reshape(-1), bits, specs, [2 * T, H, C],
                                       [0, 1, 2, -1])
    nblk = -(-T // bs)
    NB = nblk + int(rng.integers(0, 9))
    ids = rng.permutation(NB)[:nblk].astype(np.int64)
    shape = (NB, 2, bs, H, C) if blocks_first else (2, NB, bs, H, C)
    cache = rng.integers(0, 256, shape, dtype=np.uint8)
    expect = cache.copy()
    oracle.restore_layer(flat, offs, bits, specs, T, H, C, ids, expect, blocks_first)

    lay = kv_symbol_layout(T, H, C, bits, specs)
    buf = torch.zeros(flat.size + 8, dtype=torch.uint8, device=cuda_device)
    view = buf[shift:shift + flat.size]
    view.copy_(torch.from_numpy(flat).to(cuda_device))
    cache_gpu = torch.from_numpy(cache).to(cuda_device)
    ids_gpu = native_gpu.block_ids_tensor(ids, cuda_device, NB)
    native_gpu.unpack_to_kv_cache(view, lay, T, cache_gpu, ids_gpu)
    assert np.array_equal(cache_gpu.cpu().numpy(), expect), case

    out = torch.full((flat.size + 8,), 0xCD, dtype=torch.uint8, device=cuda_device)
    native_gpu.pack_from_kv_cache(cache_gpu, ids_gpu, T, lay, out[shift:shift + flat.size])
    host = out.cpu().numpy()
    assert np.array_equal(host[shift:shift + flat.size], flat), case
    assert (host[:shift] == 0xCD).all() and (host[shift + flat.size:] == 0xCD).all(), case


LAYOUTS = [
    (["token", "head", "head_dim"], [0, 1, 2, -1]),
    (["head", "token", "head_dim"], [1, 0, 2, -1]),
    (["head", "head_dim", "token"], [2, 0, 1, -1]),
    (["layer", "token", "head", "head_dim"], [1, 2, 3, 0]),
    (["token", "layer", "head_dim", "head"], [0, 3, 2, 1]),
]


@pytest.mark.parametrize("seed", range(40))
def test_random_storage_unpack_and_pack(cuda_device, seed):
    rng = np.random.default_rng(5000 + seed)
    layout, axes = LAYOUTS[seed % len(LAYOUTS)]
    T = int(rng.integers(16, 700)) if seed % 2 else 16 * int(rng.integers(1, 40))
    H = int(rng.choice([1, 2, 3, 4]))
    C = 16 * int(rng.integers(1, 9)) if seed % 4 else int(rng.integers(1, 70))
    bits = int(rng.integers(1, 9))
    shift = int(rng.choice([0, 0, 1, 2, 3]))
    kind = ["planner", "reversed", "random", "partition"][seed % 4]
    if kind == "partition":
        specs = bitref.random_specs(rng, T, H, C, partition=True)
    else:
        specs = _plan(rng, kind, T, H, C)
    shape = [{"token": T, "head": H, "head_dim": C, "layer": 1}[a] for a in layout]
    case = (layout, T, H, C, bits, shift, kind, len(specs))

    sym = rng.integers(0, 256, int(np.prod(shape)), dtype=np.uint8)
    flat, offs = oracle.pack_canonical(sym, bits, specs, shape, axes)
    ref_sym = oracle.unpack_canonical(flat, offs, bits, specs, shape, axes)

    buf = torch.zeros(flat.size + 8, dtype=torch.uint8, device=cuda_device)
    view = buf[shift:shift + flat.size]
    view.copy_(torch.from_numpy(flat).to(cuda_device))
    out = native_gpu.unpack_canonical_storage_chunks(view, bits, shape, layout, specs,
                                                     device=cuda_device)
    assert np.array_equal(out.cpu().numpy(), ref_sym), case

    lay = native_gpu.CanonicalLayout.make(shape, layout, bits, specs)
    dst = torch.full((flat.size + 8,), 0xCD, dtype=torch.uint8, device=cuda_device)
    native_gpu.pack_layout(torch.from_numpy(sym).to(cuda_device), lay,
                           dst[shift:shift + flat.size])
    host = dst.cpu().numpy()
    assert np.array_equal(host[shift:shift + flat.size], flat), case
    assert (host[:shift] == 0xCD).all() and (host[shift + flat.size:] == 0xCD).all(), case


@pytest.mark.parametrize("seed", range(30))
def test_random_cachegen_restore(cuda_device, seed):
    from tests.test_gpu_dequant import _run_both

    rng = np.random.default_rng(7000 + seed)
    heads = int(rng.integers(1, 9))
    head_dim = 8 * int(rng.integers(1, 33)) if seed % 3 else int(rng.integers(1, 70))
    tokens = int(rng.integers(1, 2000))
    bs = int(rng.choice([8, 16, 32]))
    nblk = -(-tokens // bs)
    nb = nblk + int(rng.integers(0, 6))
    kbits, vbits = int(rng.integers(2, 9)), int(rng.integers(2, 9))
    kbins = int(rng.integers(4, (1 << kbits) + 1))
    vbins = int(rng.integers(4, (1 << vbits) + 1))
    case = dict(tokens=tokens, heads=heads, head_dim=head_dim, bs=bs, nb=nb,
                ids=rng.permutation(nb)[:nblk].tolist(), key_bits=kbits, value_bits=vbits,
                key_bins=kbins, value_bins=vbins,
                out_dtype=[torch.float16, torch.bfloat16][seed % 2],
                max_dtype=[np.float16, np.float32][(seed // 2) % 2],
                blocks_first=bool(rng.integers(0, 2)), gap=int(rng.integers(0, 6)),
                cache_offset=int(rng.choice([0, 0, 0, 1])))
    got, expect = _run_both(cuda_device, rng, **case)
    assert np.array_equal(got, expect), {k: v for k, v in case.items() if k != "ids"}


@pytest.mark.parametrize("seed", range(30))
def test_random_kivi_restore(cuda_device, seed):
    from tests.test_gpu_dequant import _kivi_run_both

    rng = np.random.default_rng(9000 + seed)
    heads = int(rng.integers(1, 9))
    head_dim = 8 * int(rng.integers(1, 33)) if seed % 3 else int(rng.integers(1, 70))
    tokens = int(rng.integers(1, 1500))
    sink = int(min(tokens, rng.choice([0, 16, 24, 128])))
    bits = int(rng.integers(1, 9))
    nibble3 = bits == 3 and bool(rng.integers(0, 2))
    group = int(rng.choice([16, 32, 64, 128])) if seed % 4 else int(rng.integers(1, 100))
    bs = int(rng.choice([8, 16, 32]))
    nblk = -(-tokens // bs)
    nb = nblk + int(rng.integers(0, 6))
    case = dict(tokens=tokens, sink=sink, heads=heads, head_dim=head_dim, bits=bits,
                nibble3=nibble3, group=group, bs=bs, nb=nb,
                ids=rng.permutation(nb)[:nblk].tolist(),
                out_dtype=[torch.float16, torch.bfloat16][seed % 2],
                meta_dtype=[np.float16, np.float32][(seed // 2) % 2],
                blocks_first=bool(rng.integers(0, 2)), gap=int(rng.integers(0, 6)),
                cache_offset=int(rng.choice([0, 0, 0, 1])))
    got, expect = _kivi_run_both(cuda_device, rng, **case)
    assert np.array_equal(got, expect), {k: v for k, v in case.items() if k != "ids"}

"""Parity at token counts that move 8-bit plane runs off 128-byte lines.

For b = 8 the rows kernels read and write 16-token runs at 16-byte
boundaries.  Whether every run also starts on a 128-byte line (planes of
2T bytes with 2T % 128 == 0, the V half at byte T with T % 128 == 0) picks
non-temporal or cached accesses, and a token count that is not a multiple of
the workgroup tile's 1024 tokens leaves a partial last token tile, which the
restore orders after the full ones.  The pack of planes off the lines goes
through LDS (whole stream lines per wave) in 16-, 8- or 4-wave workgroups by
launch size; odd token counts put runs at any byte.  Each case packs one Llama-3-8B-geometry
layer (8 KV heads, head_dim 128, bf16, block size 16, permuted tables, 1 MiB
planner chunks) from the paged cache and restores it into another cache; both
must equal the oracle (chunking.py:22-123 for the plan,
bitpack_layout_cuda.cu:91-128 for the stream, benchmark_utils.py:350-444 for
the scatter), byte for byte over the whole cache."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle
from origami_amd.layout import kv_symbol_layout
from origami_amd.lossless import native_gpu
from origami_amd.lossless.chunking import plan_head_channel_chunks
from origami_amd.synthetic import fill_layer

pytestmark = pytest.mark.gpu

BS, H, D = 16, 8, 128


@pytest.fixture(scope="module", autouse=True)
def _oracle_threads():
    oracle.set_threads(min(16, os.cpu_count() or 1))


@pytest.mark.parametrize("T", [
    32784,   # planes 32 bytes off the line (2T % 128 == 32), 33 token tiles
    32832,   # planes on lines, V half 64 bytes off
    32896,   # planes and V half on lines, 128-token partial last tile
    40000,   # planes 64 bytes off, partial last tile
    49216,   # planes on lines, V half off, partial last tile
    3088,    # small: 4-wave tiles, partial last tile
    32753,   # odd: runs at any byte; staged pack in 16-wave tiles, non-temporal stores
    65521,   # odd: staged pack at 4 tiles per CU, plain stores
    12001,   # odd: staged pack, each stream line written by one tile (1 round)
    24001,   # the same over 2 rounds of tiles
    49217,   # the same over 4 rounds of tiles
    16383,   # odd: staged pack in 16-wave tiles, one per CU
    4100,    # staged pack in 8-wave tiles, 4-token last tile
    2053,    # staged pack in 4-wave tiles
])
@pytest.mark.parametrize("blocks_first", [False, True])
def test_byte_planes_off_lines(cuda_device, T, blocks_first):
    dev, C = cuda_device, D * 2
    rng = np.random.default_rng(T)
    gen = torch.Generator(device=dev)
    gen.manual_seed(T)
    nblk = -(-T // BS)
    NB = nblk + 37
    shape = (NB, 2, BS, H, D) if blocks_first else (2, NB, BS, H, D)
    src = torch.zeros(shape, dtype=torch.bfloat16, device=dev)
    if blocks_first:
        kv = torch.zeros((2, NB, BS, H, D), dtype=torch.bfloat16, device=dev)
        fill_layer(kv, torch.arange(NB, device=dev), gen)
        src.copy_(kv.transpose(0, 1))
        del kv
    else:
        fill_layer(src, torch.arange(NB, device=dev), gen)
    st = rng.permutation(NB)[:nblk].astype(np.int64)
    dt = rng.permutation(NB)[:nblk].astype(np.int64)
    plan = plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C, token_count=2 * T,
                                    bytes_per_symbol=1, min_bytes=1 << 20,
                                    target_bytes=1 << 20, max_bytes=1 << 20)
    specs = [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
              c.layout.channel_end, c.layout.token_start, c.layout.token_end] for c in plan]
    lay = kv_symbol_layout(T, H, C, 8, specs)

    stream = native_gpu.pack_from_kv_cache(src, native_gpu.block_ids_tensor(st, dev, NB), T, lay)
    src_u8 = src.view(torch.uint8).cpu().numpy()
    sym = oracle.gather_kv_cache(src_u8, st, blocks_first=blocks_first)
    sym = sym.reshape(2, -1, H, C)[:, :T].reshape(-1)
    flat, offs = oracle.pack_canonical(sym, 8, specs, [2 * T, H, C], [0, 1, 2, -1])
    assert np.array_equal(stream.cpu().numpy(), flat), "pack differs from the oracle"

    dst = torch.zeros_like(src)
    native_gpu.unpack_to_kv_cache(stream, lay, T, dst, native_gpu.block_ids_tensor(dt, dev, NB))
    expect = np.zeros_like(src_u8)
    oracle.restore_layer(flat, offs, 8, specs, T, H, C, dt, expect, blocks_first=blocks_first)
    assert np.array_equal(dst.view(torch.uint8).cpu().numpy(), expect), \
        "restore differs from the oracle"


@pytest.mark.parametrize("shift", [5, 16, 77])
@pytest.mark.parametrize("T", [32753, 24001])
def test_staged_pack_into_offset_stream(cuda_device, shift, T):
    """The staged 8-bit pack of a full layer (16-wave workgroups; at 24001
    tokens each stream line is written by one tile) written `shift` bytes
    into a larger buffer: the stream equals the oracle's and the bytes around
    it keep their guard value (the lines at the stream's ends are partial)."""
    dev, C = cuda_device, D * 2
    gen = torch.Generator(device=dev)
    gen.manual_seed(shift)
    nblk = -(-T // BS)
    NB = nblk + 11
    src = torch.zeros((2, NB, BS, H, D), dtype=torch.bfloat16, device=dev)
    fill_layer(src, torch.arange(NB, device=dev), gen)
    st = np.random.default_rng(shift).permutation(NB)[:nblk].astype(np.int64)
    plan = plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C, token_count=2 * T,
                                    bytes_per_symbol=1, min_bytes=1 << 20,
                                    target_bytes=1 << 20, max_bytes=1 << 20)
    specs = [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
              c.layout.channel_end, c.layout.token_start, c.layout.token_end] for c in plan]
    lay = kv_symbol_layout(T, H, C, 8, specs)
    buf = torch.full((lay.stream_bytes + shift + 131,), 0xA5, dtype=torch.uint8, device=dev)
    native_gpu.pack_from_kv_cache(src, native_gpu.block_ids_tensor(st, dev, NB), T, lay,
                                  buf[shift:shift + lay.stream_bytes])
    host = buf.cpu().numpy()
    sym = oracle.gather_kv_cache(src.view(torch.uint8).cpu().numpy(), st)
    sym = sym.reshape(2, -1, H, C)[:, :T].reshape(-1)
    flat, _ = oracle.pack_canonical(sym, 8, specs, [2 * T, H, C], [0, 1, 2, -1])
    assert np.array_equal(host[shift:shift + lay.stream_bytes], flat), "pack differs from the oracle"
    assert (host[:shift] == 0xA5).all() and (host[shift + lay.stream_bytes:] == 0xA5).all(), \
        "bytes outside the stream were written"


@pytest.mark.parametrize("seed", range(12))
def test_staged_pack_random_geometries(cuda_device, seed):
    """Seeded staged packs at 5000-60000 odd token counts, 2-8 heads of 128
    or 256 bytes, block sizes 8, 16, 24 or 32, both cache layouts and an output
    pointer 0-64 bytes into its buffer.  Most of these draws take 16-wave
    tiles in which each stream line is written by one tile.  The stream
    equals the oracle's and the bytes around it keep their guard value."""
    dev = cuda_device
    rng = np.random.default_rng(900 + seed)
    T = int(rng.integers(5000, 60000)) | 1
    H = int(rng.choice([2, 4, 8]))
    C = int(rng.choice([128, 256]))
    bs = int(rng.choice([8, 16, 24, 32]))
    blocks_first = bool(rng.integers(0, 2))
    shift = int(rng.choice([0, 3, 64]))
    nblk = -(-T // bs)
    NB = nblk + 9
    shape = (NB, 2, bs, H, C) if blocks_first else (2, NB, bs, H, C)
    src = torch.from_numpy(rng.integers(0, 256, shape, dtype=np.uint8)).to(dev)
    st = rng.permutation(NB)[:nblk].astype(np.int64)
    plan = plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C, token_count=2 * T,
                                    bytes_per_symbol=1, min_bytes=1 << 20,
                                    target_bytes=1 << 20, max_bytes=1 << 20)
    specs = [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
              c.layout.channel_end, c.layout.token_start, c.layout.token_end] for c in plan]
    lay = kv_symbol_layout(T, H, C, 8, specs)
    buf = torch.full((lay.stream_bytes + shift + 131,), 0xA5, dtype=torch.uint8, device=dev)
    native_gpu.pack_from_kv_cache(src, native_gpu.block_ids_tensor(st, dev, NB), T, lay,
                                  buf[shift:shift + lay.stream_bytes])
    host = buf.cpu().numpy()
    sym = oracle.gather_kv_cache(src.cpu().numpy(), st, blocks_first=blocks_first)
    sym = sym.reshape(2, -1, H, C)[:, :T].reshape(-1)
    flat, _ = oracle.pack_canonical(sym, 8, specs, [2 * T, H, C], [0, 1, 2, -1])
    case = (T, H, C, bs, blocks_first, shift)
    assert np.array_equal(host[shift:shift + lay.stream_bytes], flat), case
    assert (host[:shift] == 0xA5).all() and (host[shift + lay.stream_bytes:] == 0xA5).all(), case

"""Sub-byte packs whose plane runs start at any bit.

When T * b is not a multiple of 8 (or a plan's planes do not start on bytes),
the 16-symbol runs of a lane start inside a byte and the runs of neighbouring
lanes, waves and planes share dwords.  The rows pack then clears the stream,
stores the dwords inside an 8-lane group's runs (b >= 5) and ORs the shared
ones (every dword below b = 5) into it.  Each case packs a layer from the paged cache (the
fused save) or from a [T, H, C] symbol tensor (the storage pack) and compares
the stream with the oracle's pack (bitpack_layout_cuda.cu:70-128 for the
stream, chunking.py:22-123 for the plan), byte for byte; the bytes around an
output placed inside a larger buffer keep their guard value."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle
from origami_amd.layout import kv_symbol_layout
from origami_amd.lossless import native_gpu
from origami_amd.lossless.chunking import plan_head_channel_chunks

pytestmark = pytest.mark.gpu

H, D, BS = 8, 128, 16
C = 2 * D


@pytest.fixture(scope="module", autouse=True)
def _oracle_threads():
    oracle.set_threads(min(16, os.cpu_count() or 1))


def _specs(T2, target=1 << 20):
    return [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
             c.layout.channel_end, c.layout.token_start, c.layout.token_end]
            for c in plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C,
                                              token_count=T2, bytes_per_symbol=1,
                                              min_bytes=target, target_bytes=target,
                                              max_bytes=target)]


@pytest.mark.parametrize("T,bits,shift", [
    (4099, 7, 0),    # odd T: runs at any bit
    (4100, 3, 0),    # even T, T * b % 8 == 4
    (2053, 1, 3),    # b = 1: a dword holds bits of three runs; stream 3 bytes into a buffer
    (2053, 5, 1),
    (8198, 6, 2),    # T * b % 8 == 4 at b = 6
    (4098, 2, 0),    # b = 2, T * b % 8 == 4
    (2053, 4, 5),    # b = 4, odd T
    (32753, 7, 0),   # a full Llama-3-8B layer, 16-wave tiles
])
def test_fused_save_runs_at_any_bit(cuda_device, T, bits, shift):
    dev = cuda_device
    rng = np.random.default_rng(T * 10 + bits)
    nblk = -(-T // BS)
    NB = nblk + 5
    cache_u8 = rng.integers(0, 1 << bits, (2, NB, BS, H, C), dtype=np.uint8)
    cache = torch.from_numpy(cache_u8).to(dev).view(torch.bfloat16)
    table = rng.permutation(NB)[:nblk].astype(np.int64)
    specs = _specs(2 * T)
    lay = kv_symbol_layout(T, H, C, bits, specs)
    buf = torch.full((lay.stream_bytes + shift + 67,), 0xA5, dtype=torch.uint8, device=dev)
    native_gpu.pack_from_kv_cache(cache, native_gpu.block_ids_tensor(table, dev, NB), T, lay,
                                  buf[shift:shift + lay.stream_bytes])
    sym = oracle.gather_kv_cache(cache_u8, table).reshape(2, -1, H, C)[:, :T].reshape(-1)
    flat, _ = oracle.pack_canonical(sym, bits, specs, [2 * T, H, C], [0, 1, 2, -1])
    host = buf.cpu().numpy()
    assert np.array_equal(host[shift:shift + lay.stream_bytes], flat), "pack differs from the oracle"
    assert (host[:shift] == 0xA5).all() and (host[shift + lay.stream_bytes:] == 0xA5).all(), \
        "bytes outside the stream were written"


@pytest.mark.parametrize("T,bits,shift", [(4099, 7, 1), (2053, 3, 0)])
def test_fused_save_into_larger_output(cuda_device, T, bits, shift):
    """An output buffer longer than the stream: the pack writes the stream's
    bytes only, and the buffer's tail past them keeps its guard value."""
    dev = cuda_device
    rng = np.random.default_rng(T * 7 + bits)
    nblk = -(-T // BS)
    NB = nblk + 3
    cache_u8 = rng.integers(0, 1 << bits, (2, NB, BS, H, C), dtype=np.uint8)
    cache = torch.from_numpy(cache_u8).to(dev).view(torch.bfloat16)
    table = rng.permutation(NB)[:nblk].astype(np.int64)
    specs = _specs(2 * T)
    lay = kv_symbol_layout(T, H, C, bits, specs)
    buf = torch.full((lay.stream_bytes + shift + 4099,), 0x5A, dtype=torch.uint8, device=dev)
    native_gpu.pack_from_kv_cache(cache, native_gpu.block_ids_tensor(table, dev, NB), T, lay,
                                  buf[shift:])
    sym = oracle.gather_kv_cache(cache_u8, table).reshape(2, -1, H, C)[:, :T].reshape(-1)
    flat, _ = oracle.pack_canonical(sym, bits, specs, [2 * T, H, C], [0, 1, 2, -1])
    host = buf.cpu().numpy()
    assert np.array_equal(host[shift:shift + lay.stream_bytes], flat), "pack differs from the oracle"
    assert (host[:shift] == 0x5A).all() and (host[shift + lay.stream_bytes:] == 0x5A).all(), \
        "bytes outside the stream were written"


@pytest.mark.parametrize("T,bits,target", [(2051, 3, 1 << 15), (1027, 7, 1 << 14), (4096, 5, 3000)])
def test_storage_pack_runs_at_any_bit(cuda_device, T, bits, target):
    """A [T, H, C] symbol tensor packed with small chunks (planes split
    across chunks); 3000-byte chunks at T = 4096 leave planes off bytes
    even though T * b is a multiple of 8."""
    dev = cuda_device
    rng = np.random.default_rng(T + bits)
    specs = [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
              c.layout.channel_end, c.layout.token_start, c.layout.token_end]
             for c in plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C,
                                               token_count=T, bytes_per_symbol=1,
                                               min_bytes=target, target_bytes=target,
                                               max_bytes=target)]
    sym = rng.integers(0, 1 << bits, T * H * C, dtype=np.uint8)
    flat, _ = oracle.pack_canonical(sym, bits, specs, [T, H, C], [0, 1, 2, -1])
    chunks = native_gpu.pack_canonical_storage_chunks(
        torch.from_numpy(sym.reshape(T, H, C)).to(dev), bits, [T, H, C],
        ["token", "head", "head_dim"], specs)
    got = np.concatenate([c.cpu().numpy() for c in chunks])
    assert np.array_equal(got, flat)

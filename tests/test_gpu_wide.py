"""Restores at b = 1, 2 and 4 whose lane runs are whole 16-byte chunks.

When every plane starts on a 16-byte boundary, the stream pointer is 16-byte
aligned and the token count is a multiple of 128 / b, a lane of the restore
reads one 16-byte chunk per plane (128 / b tokens) and restores it as
16-token sub-tiles.  Non-temporal loads when every 8-lane group reads one
128-byte line (T * b a multiple of 1024), cached loads otherwise; token counts
that are not a multiple of 128 / b, and misaligned streams, take the window or
shift modes.  Each case restores a layer packed by the oracle
(bitpack_layout_cuda.cu:70-128 for the stream, benchmark_utils.py:350-444 for
the scatter) into a paged cache holding random bytes, and compares the whole
cache byte for byte with the oracle's restore; the storage-layout unpack
(a [T, H, C] symbol tensor) is compared with the oracle's unpack."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle
from origami_amd.layout import kv_symbol_layout
from origami_amd.lossless import native_gpu
from origami_amd.lossless.chunking import plan_head_channel_chunks

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _oracle_threads():
    oracle.set_threads(min(16, os.cpu_count() or 1))


def _specs(T2, H, C, target):
    return [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
             c.layout.channel_end, c.layout.token_start, c.layout.token_end]
            for c in plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C,
                                              token_count=T2, bytes_per_symbol=1,
                                              min_bytes=target, target_bytes=target,
                                              max_bytes=target)]


def _restore_case(dev, T, H, C, bits, bs=16, blocks_first=False, shift=0, target=1 << 20,
                  seed=0):
    rng = np.random.default_rng(seed)
    specs = _specs(2 * T, H, C, target)
    value = rng.integers(0, 1 << bits, (2, T, H, C), dtype=np.uint8)
    flat, offs = oracle.pack_canonical(value.reshape(-1), bits, specs, [2 * T, H, C],
                                       [0, 1, 2, -1])
    nblk = -(-T // bs)
    NB = nblk + 7
    ids = rng.permutation(NB)[:nblk].astype(np.int64)
    shape = (NB, 2, bs, H, C) if blocks_first else (2, NB, bs, H, C)
    cache = rng.integers(0, 256, shape, dtype=np.uint8)
    expect = cache.copy()
    oracle.restore_layer(flat, offs, bits, specs, T, H, C, ids, expect, blocks_first)

    lay = kv_symbol_layout(T, H, C, bits, specs)
    buf = torch.zeros(flat.size + 256, dtype=torch.uint8, device=dev)
    view = buf[shift:shift + flat.size]
    view.copy_(torch.from_numpy(flat).to(dev))
    got = torch.from_numpy(cache).to(dev)
    native_gpu.unpack_to_kv_cache(view, lay, T, got, native_gpu.block_ids_tensor(ids, dev, NB))
    assert np.array_equal(got.cpu().numpy(), expect), (T, H, C, bits, bs, blocks_first, shift)


@pytest.mark.parametrize("bits", [1, 2, 4])
@pytest.mark.parametrize("blocks_first", [False, True])
def test_wide_runs_on_lines(cuda_device, bits, blocks_first):
    # T * b % 1024 == 0: non-temporal 16-byte runs, every group on one line
    _restore_case(cuda_device, 4096, 8, 256, bits, blocks_first=blocks_first, seed=bits)


@pytest.mark.parametrize("bits", [1, 2, 4])
def test_wide_runs_off_lines(cuda_device, bits):
    # T a multiple of 128 / b but T * b not of 1024: cached 16-byte runs; the
    # last token tile is partial and rows past T in its last block are zeroed
    _restore_case(cuda_device, 4096 + 128 // bits, 8, 256, bits, bs=32, seed=10 + bits)


@pytest.mark.parametrize("bits,T,bs,blocks_first", [
    (4, 4096, 8, False),              # on lines, a lane's 16-row sub-tiles span two blocks
    (2, 4096, 24, True),              # on lines, sub-tiles cross 24-row block boundaries
    (1, 4096, 24, False),
    (4, 4096 + 32, 24, False),        # off lines (cached runs), partial last block
    (2, 4096 + 64, 8, True),
    (1, 4096 + 128, 8, False),
])
def test_wide_runs_block_sizes_off_16(cuda_device, bits, T, bs, blocks_first):
    # block sizes that are not a multiple of 16: the row stores follow the
    # block table row by row
    _restore_case(cuda_device, T, 8, 256, bits, bs=bs, blocks_first=blocks_first,
                  seed=70 + bits + bs)


@pytest.mark.parametrize("bits,T", [(4, 4096 + 16), (2, 4096 + 32), (1, 4096 + 64)])
def test_token_count_off_the_run_falls_back(cuda_device, bits, T):
    _restore_case(cuda_device, T, 8, 256, bits, seed=20 + bits)


@pytest.mark.parametrize("bits", [1, 2, 4])
def test_misaligned_stream_falls_back(cuda_device, bits):
    _restore_case(cuda_device, 4096, 4, 256, bits, shift=4, seed=30 + bits)


@pytest.mark.parametrize("bits", [1, 2, 4])
def test_partial_channel_groups_and_small_chunks(cuda_device, bits):
    # 2 heads x 48 bytes: 6 of a wave's 8 channel groups hold planes; 16 KiB
    # chunks cut the planes into many chunks
    _restore_case(cuda_device, 2048, 2, 48, bits, target=1 << 14, seed=40 + bits)


def test_wide_runs_full_layer(cuda_device):
    # Llama-3-8B geometry at b = 4: 32768 tokens, 8 heads x 256 bytes
    _restore_case(cuda_device, 32768, 8, 256, 4, seed=50)


@pytest.mark.parametrize("bits", [1, 2, 4])
def test_wide_storage_unpack(cuda_device, bits):
    dev = cuda_device
    rng = np.random.default_rng(60 + bits)
    T, H, C = 2048, 4, 128
    specs = _specs(T, H, C, 1 << 15)
    sym = rng.integers(0, 1 << bits, T * H * C, dtype=np.uint8)
    flat, offs = oracle.pack_canonical(sym, bits, specs, [T, H, C], [0, 1, 2, -1])
    ref = oracle.unpack_canonical(flat, offs, bits, specs, [T, H, C], [0, 1, 2, -1])
    buf = torch.zeros(flat.size + 256, dtype=torch.uint8, device=dev)
    buf[:flat.size].copy_(torch.from_numpy(flat).to(dev))
    out = native_gpu.unpack_canonical_storage_chunks(buf[:flat.size], bits, [T, H, C],
                                                     ["token", "head", "head_dim"], specs,
                                                     device=dev)
    assert np.array_equal(out.cpu().numpy(), ref)

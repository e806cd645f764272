"""The single-layer Llama-3-8B workload end to end: 8 KV heads, head_dim 128,
4096 tokens, block_size 16, bf16; K = N(0,1) times a per-channel
LogNormal(0,1) scale with 4 outlier channels per head x20, V = N(0, 0.5);
torch CPU generator seed 0.  The layer is packed to the codec layout
(1 MiB planner chunks, chunking.py:22-123; plane-major stream,
bitpack_layout_cuda.cu:70-128), each chunk goes through the CPU codec's
zlib level-1 raw-deflate round trip (cpu_qat.py:64-83), and the stream is
unpacked and scattered into a contiguous block table 0..255
(benchmark_utils.py:350-444).  Checked bit-exact against the source
blocks.  The CPU case runs the oracle's pack and restore; the GPU case runs
the HIP fused save and restore and compares every stage with the oracle."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle
from origami_amd.layout import kv_symbol_layout
from origami_amd.lossless.chunking import plan_head_channel_chunks
from origami_amd.lossless.cpu_qat import CpuLosslessCodec
from origami_amd.synthetic import fill_layer

T, H, D, BS = 4096, 8, 128, 16
C = 2 * D
NBLK = T // BS


@pytest.fixture(scope="module", autouse=True)
def _oracle_threads():
    oracle.set_threads(min(16, os.cpu_count() or 1))


def _workload():
    gen = torch.Generator().manual_seed(0)
    cache = torch.zeros((2, NBLK, BS, H, D), dtype=torch.bfloat16)
    fill_layer(cache, torch.arange(NBLK), gen)
    specs = [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
              c.layout.channel_end, c.layout.token_start, c.layout.token_end]
             for c in plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C,
                                               token_count=2 * T, bytes_per_symbol=1,
                                               min_bytes=1 << 20, target_bytes=1 << 20,
                                               max_bytes=1 << 20)]
    return cache, specs


def _zlib_round_trip(stream: np.ndarray, offsets: np.ndarray) -> np.ndarray:
    codec = CpuLosslessCodec(backend="zlib", threads=4)
    chunks = [torch.from_numpy(stream[int(a):int(b)].copy())
              for a, b in zip(offsets[:-1], offsets[1:])]
    comp = codec.compress_many(chunks)
    assert sum(int(c.numel()) for c in comp) < stream.size  # the K/V bytes compress
    back = codec.decompress_many(comp, [int(c.numel()) for c in chunks])
    return torch.cat(back).numpy()


def test_c1_workload_oracle_path():
    cache, specs = _workload()
    src = cache.view(torch.uint8).numpy()
    assert len(specs) == 16  # 2 chunks of 1 MiB per head
    ids = np.arange(NBLK, dtype=np.int64)
    sym = oracle.gather_kv_cache(src, ids).reshape(-1)
    stream, offs = oracle.pack_canonical(sym, 8, specs, [2 * T, H, C], [0, 1, 2, -1])
    # plane-major transpose of the token-major K/V bytes (bits 8)
    assert np.array_equal(stream.reshape(H * C, 2 * T), sym.reshape(2 * T, H * C).T)
    back = _zlib_round_trip(stream, offs)
    assert np.array_equal(back, stream)
    out = np.zeros_like(src)
    oracle.restore_layer(back, offs, 8, specs, T, H, C, ids, out)
    assert np.array_equal(out, src)


@pytest.mark.gpu
def test_c1_workload_hip_path(cuda_device):
    from origami_amd.lossless import native_gpu

    cache, specs = _workload()
    src = cache.view(torch.uint8).numpy()
    lay = kv_symbol_layout(T, H, C, 8, specs)
    ids = torch.arange(NBLK, dtype=torch.int64, device=cuda_device)
    stream = native_gpu.pack_from_kv_cache(cache.to(cuda_device), ids, T, lay).cpu().numpy()
    sym = oracle.gather_kv_cache(src, ids.cpu().numpy()).reshape(-1)
    ref, offs = oracle.pack_canonical(sym, 8, specs, [2 * T, H, C], [0, 1, 2, -1])
    assert np.array_equal(stream, ref), "pack differs from the oracle"
    back = _zlib_round_trip(stream, offs)
    dst = torch.zeros((2, NBLK, BS, H, D), dtype=torch.bfloat16, device=cuda_device)
    native_gpu.unpack_to_kv_cache(torch.from_numpy(back).to(cuda_device), lay, T, dst, ids)
    got = dst.view(torch.uint8).cpu().numpy()
    expect = np.zeros_like(src)
    oracle.restore_layer(back, offs, 8, specs, T, H, C, ids.cpu().numpy(), expect)
    assert np.array_equal(got, expect), "restore differs from the oracle"
    assert np.array_equal(got, src), "restored blocks differ from the source"

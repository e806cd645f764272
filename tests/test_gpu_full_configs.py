"""Full-size oracle parity at the benchmark geometries (one layer each):

* Qwen2.5-7B batch: 4 KV heads, head_dim 128, bf16, block size 16; 8
  requests with lengths default_rng(2).integers(8192, 65537, 8); each
  request's first floor(T/2/16) blocks come from a prefix pool shared by all
  block tables (in the source and in the destination cache);
* Llama-3-8B fp8 e4m3: 8 KV heads, head_dim 128 (128-byte head rows), 16
  requests of 16384 tokens, seed 3;
* Llama-3-70B geometry: one 131072-token bf16 layer, 512 chunks of 1 MiB,
  permuted block table, seed 4 (stream bit offsets pass 2**32);
* one TP = 8 rank's share of the 32768-token Llama-3-8B layer: 1 KV head.

Chunks come from the planner at 1 MiB (chunking.py:22-123).  For every
request the HIP pack from the paged cache must equal the oracle's pack of
the gathered bytes, and the HIP restore into the destination cache must
equal the oracle's unpack + scatter (benchmark_utils.py:350-444), over the
whole cache, byte for byte.  For the two batches, the batched restore (one
launch per layer, shared prefix blocks written once) must give the same
cache."""
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

BS = 16


@pytest.fixture(scope="module", autouse=True)
def _oracle_threads():
    oracle.set_threads(min(16, os.cpu_count() or 1))


def _layout(T, H, C):
    plan = plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C, token_count=2 * T,
                                    bytes_per_symbol=1, min_bytes=1 << 20,
                                    target_bytes=1 << 20, max_bytes=1 << 20)
    specs = [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
              c.layout.channel_end, c.layout.token_start, c.layout.token_end] for c in plan]
    return kv_symbol_layout(T, H, C, 8, specs)


def _tables(perm, nblks, shared, pool):
    cur, out = pool, []
    for n, k in zip(nblks, shared):
        out.append(np.concatenate([perm[:k], perm[cur:cur + n - k]]).astype(np.int64))
        cur += n - k
    return out


def _run(dev, H, D, dtype, lengths, seed, shared_pool, expect_chunks=None, batch=False, bs=BS):
    esize = torch.empty((), dtype=dtype).element_size()
    C = D * esize
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    nblks = [-(-int(T) // bs) for T in lengths]
    shared = [int(T) // 2 // bs if shared_pool else 0 for T in lengths]
    pool = max(shared) if shared_pool else 0
    NB = pool + sum(n - k for n, k in zip(nblks, shared)) + 64
    src = torch.zeros((2, NB, bs, H, D), dtype=dtype, device=dev)
    fill_layer(src, torch.arange(NB, device=dev), gen)
    src_tables = _tables(rng.permutation(NB), nblks, shared, pool)
    dst_tables = _tables(rng.permutation(NB), nblks, shared, pool)
    dst = torch.zeros_like(src)
    src_u8 = src.view(torch.uint8).cpu().numpy()
    expect = np.zeros_like(src_u8)
    layouts = {}
    streams = []
    for T, st, dt in zip(lengths, src_tables, dst_tables):
        T = int(T)
        lay = layouts.setdefault(T, _layout(T, H, C))
        if expect_chunks is not None:
            assert lay.num_chunks == expect_chunks
        stream = native_gpu.pack_from_kv_cache(src, native_gpu.block_ids_tensor(st, dev, NB), T,
                                               lay)
        sym = oracle.gather_kv_cache(src_u8, st).reshape(2, -1, H, C)[:, :T].reshape(-1)
        flat, offs = oracle.pack_canonical(sym, 8, lay.specs, [2 * T, H, C], [0, 1, 2, -1])
        del sym
        assert np.array_equal(stream.cpu().numpy(), flat), f"pack differs at T={T}"
        native_gpu.unpack_to_kv_cache(stream, lay, T, dst,
                                      native_gpu.block_ids_tensor(dt, dev, NB))
        oracle.restore_layer(flat, offs, 8, lay.specs, T, H, C, dt, expect)
        if batch:
            streams.append(stream)
        del flat, stream
    got = dst.view(torch.uint8).cpu().numpy()
    assert np.array_equal(got, expect), "restored cache differs from the oracle"
    if batch:
        # one launch per layer for the whole batch, shared prefix blocks once
        dst.zero_()
        native_gpu.unpack_batch_to_kv_cache(
            [(s_, layouts[int(T)], int(T), dt) for s_, T, dt in zip(streams, lengths, dst_tables)],
            dst, dedup_shared_blocks=shared_pool)
        assert np.array_equal(dst.view(torch.uint8).cpu().numpy(), expect), \
            "batched restore differs from the oracle"
        del streams
    # and from the source blocks themselves (the prefix pool holds identical
    # bytes for every request that references it)
    for T, st, dt in zip(lengths, src_tables, dst_tables):
        a = got[:, dt].reshape(2, -1, H, C)[:, :int(T)]
        b = src_u8[:, st].reshape(2, -1, H, C)[:, :int(T)]
        assert np.array_equal(a, b)
    return NB, dst_tables


def test_qwen25_7b_batch_full(cuda_device):
    lengths = np.random.default_rng(2).integers(8192, 65537, 8)
    assert not all(int(T) % 16 == 0 for T in lengths)  # ragged lengths are covered
    NB, tables = _run(cuda_device, 4, 128, torch.bfloat16, lengths, 2, True, batch=True)
    # the destination prefix pool is referenced by every table
    k = min(int(T) // 2 // BS for T in lengths)
    assert all(np.array_equal(t[:k], tables[0][:k]) for t in tables)


def test_llama3_8b_fp8_16x16k_full(cuda_device):
    _run(cuda_device, 8, 128, torch.float8_e4m3fn, [16384] * 16, 3, False, expect_chunks=32,
         batch=True)


def test_llama3_70b_131072_full(cuda_device):
    _run(cuda_device, 8, 128, torch.bfloat16, [131072], 4, False, expect_chunks=512)


@pytest.mark.parametrize("T", [32768, 32753])
def test_llama3_8b_tp8_rank_share_full(cuda_device, T):
    """One tensor-parallel rank's share of the 32768-token Llama-3-8B layer
    at TP = 8 (config.py:312-320 gives each rank its own KV heads): 1 KV
    head, head_dim 128, bf16 (256-byte rows), 16 chunks of 1 MiB, permuted
    block table; and the same at a ragged length."""
    _run(cuda_device, 1, 128, torch.bfloat16, [T], 8, False,
         expect_chunks=16 if T == 32768 else None)


def test_batch_split_launch_block_size_24(cuda_device):
    """The fp8 batch (16 x 16384 tokens, 4-wave workgroups per tile) with
    24-token blocks and a shared prefix pool: a lane's 16 rows cross block
    boundaries, so the restore follows the block table row by row."""
    _run(cuda_device, 8, 128, torch.float8_e4m3fn, [16384] * 16, 5, True, batch=True, bs=24)


@pytest.mark.parametrize("T,bits,bs", [(131067, 8, 16), (131072, 4, 16), (131072, 3, 16),
                                       (131061, 5, 16), (131072, 8, 24), (131061, 4, 8)])
def test_large_single_request_split_launch(cuda_device, T, bits, bs):
    """One ~131072-token layer (8 heads, 256-byte head rows, 2048 tiles: the
    restore launch that dispatches each tile as 4-wave workgroups) in the
    shift (ragged T) and window (sub-byte widths) addressing modes, against the
    oracle's unpack + scatter of the oracle's pack.  With 16-token blocks a
    lane's 16 rows lie in one block; 24- and 8-token blocks take the
    row-by-row walk of the block table."""
    _restore_random_layer(cuda_device, T, bits, bs)


@pytest.mark.parametrize("T,bits,bs", [
    (32753, 7, 16),   # 16-wave tiles, 16 waves per CU: plane loads one plane at a time
    (32753, 8, 24),   # the same with the block-table walk
    (15000, 8, 16),   # 4-wave tiles, ~15 waves per CU: serial plane loads
    (8200, 8, 16),    # ~8 waves per CU: every plane load in flight, block-table walk
    (4100, 7, 16),    # ~4 waves per CU: one block per lane
    (4100, 5, 8),     # the same launch size with 8-token blocks
])
def test_restore_orders_by_launch_size(cuda_device, T, bits, bs):
    """Whole-tile restores whose launch size picks the order of plane loads
    and row stores (the results must not depend on it)."""
    _restore_random_layer(cuda_device, T, bits, bs)


def test_batch_serial_plane_loads(cuda_device):
    """A batch of four ragged ~8000-token requests in 16-wave tiles (512
    tiles, one launch with 16 waves per CU)."""
    _run(cuda_device, 8, 128, torch.bfloat16, [8001, 7999, 8003, 7995], 6, False, batch=True)


def _restore_random_layer(dev, T, bits, bs):
    H, C = 8, 256
    rng = np.random.default_rng(T + bits)
    plan = plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C, token_count=2 * T,
                                    bytes_per_symbol=1, min_bytes=1 << 20,
                                    target_bytes=1 << 20, max_bytes=1 << 20)
    specs = [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
              c.layout.channel_end, c.layout.token_start, c.layout.token_end] for c in plan]
    lay = kv_symbol_layout(T, H, C, bits, specs)
    sym = rng.integers(0, 256, 2 * T * H * C, dtype=np.uint8)
    flat, offs = oracle.pack_canonical(sym, bits, specs, [2 * T, H, C], [0, 1, 2, -1])
    del sym
    nblk = -(-T // bs)
    NB = nblk + 64
    table = rng.permutation(NB)[:nblk].astype(np.int64)
    dst = torch.zeros((2, NB, bs, H, C // 2), dtype=torch.bfloat16, device=dev)
    native_gpu.unpack_to_kv_cache(torch.from_numpy(flat).to(dev), lay, T, dst,
                                  native_gpu.block_ids_tensor(table, dev, NB))
    expect = np.zeros((2, NB, bs, H, C), dtype=np.uint8)
    oracle.restore_layer(flat, offs, bits, specs, T, H, C, table, expect)
    assert np.array_equal(dst.view(torch.uint8).cpu().numpy(), expect.reshape(2, NB, bs, H, C))

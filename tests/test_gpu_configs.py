"""Benchmark-configuration-shaped parity cases (scaled to test sizes):

* Qwen2.5-7B KV geometry (4 KV heads, head_dim 128, bf16): a batch of
  requests with random lengths whose first half of blocks comes from a shared
  prefix pool referenced by several block tables (identical bytes restored
  more than once);
* Llama-3-8B geometry with an fp8 e4m3 KV cache (1-byte elements, 128 bytes
  per head) and several requests.

Everything is compared byte for byte with the oracle."""
import numpy as np
import pytest
import torch

from oracle import oracle
from origami_amd.layout import kv_symbol_layout
from origami_amd.lossless import native_gpu
from origami_amd.lossless.chunking import plan_head_channel_chunks
from origami_amd.synthetic import fill_layer

pytestmark = pytest.mark.gpu


def _specs(T2, H, C, target=1 << 18):
    return [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
             c.layout.channel_end, 0, T2]
            for c in plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C,
                                              token_count=T2, bytes_per_symbol=1,
                                              min_bytes=target, target_bytes=target,
                                              max_bytes=target)]


def test_qwen_batch_with_shared_prefix(cuda_device):
    rng = np.random.default_rng(2)
    g = torch.Generator(device=cuda_device).manual_seed(2)
    H, D, bs, nreq = 4, 128, 16, 8
    C = 2 * D
    lengths = rng.integers(500, 4000, nreq)          # ragged, not multiples of 16
    shared_blocks = int(lengths.min() // 2 // bs)    # common prefix, in blocks
    NB = 2048
    src = torch.zeros((2, NB, bs, H, D), dtype=torch.bfloat16, device=cuda_device)
    perm = rng.permutation(NB)
    prefix = perm[:shared_blocks]
    cursor = shared_blocks
    tables = []
    for T in lengths:
        n = -(-int(T) // bs)
        own = perm[cursor:cursor + n - shared_blocks]
        cursor += n - shared_blocks
        tables.append(np.concatenate([prefix, own]).astype(np.int64))
    all_ids = torch.from_numpy(np.unique(np.concatenate(tables))).to(cuda_device)
    fill_layer(src, all_ids, g)

    dst = torch.zeros_like(src)
    dperm = rng.permutation(NB)
    dprefix = dperm[:shared_blocks]
    dcur = shared_blocks
    dtables = []
    for T in lengths:
        n = -(-int(T) // bs)
        own = dperm[dcur:dcur + n - shared_blocks]
        dcur += n - shared_blocks
        dtables.append(np.concatenate([dprefix, own]).astype(np.int64))

    expect = np.zeros((2, NB, bs, H, C), np.uint8)
    src_u8 = src.view(torch.uint8).cpu().numpy()
    for T, st, dt in zip(lengths, tables, dtables):
        T = int(T)
        lay = kv_symbol_layout(T, H, C, 8, _specs(2 * T, H, C))
        stream = native_gpu.pack_from_kv_cache(src, native_gpu.block_ids_tensor(st, cuda_device),
                                               T, lay)
        native_gpu.unpack_to_kv_cache(stream, lay, T, dst,
                                      native_gpu.block_ids_tensor(dt, cuda_device))
        # oracle: gather the request's tokens, pack, unpack + scatter
        sym = oracle.gather_kv_cache(src_u8, st).reshape(2, -1, H, C)[:, :T].reshape(-1)
        flat, offs = oracle.pack_canonical(sym, 8, lay.specs, [2 * T, H, C], [0, 1, 2, -1])
        assert np.array_equal(stream.cpu().numpy(), flat)
        oracle.restore_layer(flat, offs, 8, lay.specs, T, H, C, dt, expect)
    got = dst.view(torch.uint8).cpu().numpy()
    # shared prefix blocks were restored once per request with identical bytes
    assert np.array_equal(got, expect)
    for T, st, dt in zip(lengths, tables, dtables):
        a = got[:, dt].reshape(2, -1, H, C)[:, :int(T)]
        b = src_u8[:, st].reshape(2, -1, H, C)[:, :int(T)]
        assert np.array_equal(a, b)


def test_fp8_e4m3_requests(cuda_device):
    g = torch.Generator(device=cuda_device).manual_seed(3)
    rng = np.random.default_rng(3)
    H, D, bs, T, nreq = 8, 128, 16, 2048, 4
    nblk = T // bs
    NB = nreq * nblk + 32
    src = torch.zeros((2, NB, bs, H, D), dtype=torch.float8_e4m3fn, device=cuda_device)
    dst = torch.zeros_like(src)
    perm = rng.permutation(NB)
    dperm = rng.permutation(NB)
    lay = kv_symbol_layout(T, H, D, 8, _specs(2 * T, H, D, 1 << 17))
    assert lay.num_chunks == 8 * 4  # 4 chunks per head of 32 channels
    for r in range(nreq):
        sid = torch.from_numpy(perm[r * nblk:(r + 1) * nblk]).to(cuda_device)
        did = torch.from_numpy(dperm[r * nblk:(r + 1) * nblk]).to(cuda_device)
        fill_layer(src, sid, g)
        stream = native_gpu.pack_from_kv_cache(src, sid, T, lay)
        sym = oracle.gather_kv_cache(src.view(torch.uint8).cpu().numpy(), sid.cpu().numpy())
        flat, _ = oracle.pack_canonical(sym, 8, lay.specs, [2 * T, H, D], [0, 1, 2, -1])
        assert np.array_equal(stream.cpu().numpy(), flat)
        native_gpu.unpack_to_kv_cache(stream, lay, T, dst, did)
        assert torch.equal(dst[:, did].view(torch.uint8), src[:, sid].view(torch.uint8))

"""Batched fused restore (one layer of several requests, one launch per symbol
width and addressing mode; 8-bit requests with and without 128-byte-line runs
share a launch): byte for byte the result of restoring the
requests one after another, and of the oracle's unpack + scatter in the same
order, across ragged and aligned lengths, widths, more requests than one
launch holds, both cache layouts, block sizes, shared prefix blocks (written
once under dedup) and a shared partial block (request-by-request fallback)."""
import numpy as np
import pytest
import torch

from oracle import oracle
from origami_amd.layout import kv_symbol_layout
from origami_amd.lossless import native_gpu
from origami_amd.lossless.chunking import plan_head_channel_chunks

pytestmark = pytest.mark.gpu


def _layout(T, H, C, bits, target=1 << 15):
    plan = plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C, token_count=2 * T,
                                    bytes_per_symbol=1, min_bytes=target, target_bytes=target,
                                    max_bytes=target)
    specs = [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
              c.layout.channel_end, 0, 2 * T] for c in plan]
    return kv_symbol_layout(T, H, C, bits, specs)


def _tables(rng, NB, nblks, shared):
    perm = rng.permutation(NB)
    cur, out = max(shared) if shared else 0, []
    for n, k in zip(nblks, shared):
        out.append(np.concatenate([perm[:k], perm[cur:cur + n - k]]).astype(np.int64))
        cur += n - k
    return out


def _run(dev, rng, lengths, H, C, bits, bs, blocks_first, shared_frac, dedup,
         partial_conflict=False, interior_share=False):
    nblks = [-(-int(T) // bs) for T in lengths]
    shared = [int(int(T) * shared_frac) // bs for T in lengths]
    NB = sum(nblks) + 16
    dst_tables = _tables(rng, NB, nblks, shared)
    if partial_conflict:
        # request 1's partial last block is also a block of request 0
        assert int(lengths[1]) % bs != 0
        dst_tables[1][-1] = dst_tables[0][-1 if int(lengths[0]) % bs == 0 else 0]
    # prefix bytes are the same in every request that shares the prefix
    prefix_sym = rng.integers(0, 256, (2, max(shared + [0]) * bs, H, C), dtype=np.uint8)
    shared_mid = None
    if interior_share:
        # block 3 of request 1 is block 5 of request 0, with the same bytes
        dst_tables[1][3] = dst_tables[0][5]
        shared_mid = rng.integers(0, 256, (2, bs, H, C), dtype=np.uint8)
    items, host = [], []
    for i, (T, k) in enumerate(zip(lengths, shared)):
        T = int(T)
        sym = rng.integers(0, 256, (2, T, H, C), dtype=np.uint8)
        sym[:, :k * bs] = prefix_sym[:, :k * bs]
        if shared_mid is not None and i in (0, 1):
            at = (5 if i == 0 else 3) * bs
            sym[:, at:at + bs] = shared_mid
        lay = _layout(T, H, C, bits)
        flat, offs = oracle.pack_canonical(sym.reshape(-1), bits, lay.specs, [2 * T, H, C],
                                           [0, 1, 2, -1])
        items.append((torch.from_numpy(flat).to(dev), lay, T))
        host.append((flat, offs, lay, T))
    shape = (NB, 2, bs, H, C) if blocks_first else (2, NB, bs, H, C)
    seq = torch.full(shape, 0x33, dtype=torch.uint8, device=dev)
    bat = torch.full_like(seq, 0x33)
    expect = np.full(shape, 0x33, dtype=np.uint8)
    for (flat, lay, T), t, (hf, ho, hl, _) in zip(items, dst_tables, host):
        native_gpu.unpack_to_kv_cache(flat, lay, T, seq, torch.from_numpy(t).to(dev))
        oracle.restore_layer(hf, ho, bits, hl.specs, T, H, C, t, expect,
                             blocks_first=blocks_first)
    native_gpu.unpack_batch_to_kv_cache(
        [(flat, lay, T, t) for (flat, lay, T), t in zip(items, dst_tables)], bat,
        dedup_shared_blocks=dedup)
    torch.cuda.synchronize(dev)
    s, b = seq.cpu().numpy(), bat.cpu().numpy()
    assert np.array_equal(s, expect), "sequential restore differs from the oracle"
    assert np.array_equal(b, expect), "batched restore differs from the oracle"


@pytest.mark.parametrize("dedup", [False, True])
@pytest.mark.parametrize("bits", [8, 4, 3])
def test_batch_ragged_shared_prefix(cuda_device, bits, dedup):
    rng = np.random.default_rng(40 + bits)
    lengths = rng.integers(200, 3000, 6)
    _run(cuda_device, rng, lengths, 4, 256, bits, 16, False, 0.5, dedup)


def test_batch_more_requests_than_one_launch(cuda_device):
    rng = np.random.default_rng(3)
    lengths = [int(x) * 16 for x in rng.integers(20, 200, 19)] + [777, 1001, 64]
    _run(cuda_device, rng, lengths, 8, 128, 8, 16, False, 0.0, False)


@pytest.mark.parametrize("bits", [8, 5, 1])
@pytest.mark.parametrize("blocks_first", [False, True])
def test_batch_tiny_requests(cuda_device, bits, blocks_first):
    """Requests of 1 to 33 tokens (every lane run partial or the stream ending
    inside it) beside one of 1500, in one batch, with and without a shared
    prefix of whole blocks."""
    rng = np.random.default_rng(70 + bits + int(blocks_first))
    lengths = [1, 5, 15, 16, 17, 33, 1500]
    _run(cuda_device, rng, lengths, 2, 64, bits, 16, blocks_first, 0.0, False)
    _run(cuda_device, rng, [32, 33, 48, 1500], 2, 64, bits, 16, blocks_first, 0.5, True)


@pytest.mark.parametrize("bs,blocks_first", [(32, True), (8, False), (16, True)])
def test_batch_block_sizes_and_layouts(cuda_device, bs, blocks_first):
    rng = np.random.default_rng(bs + int(blocks_first))
    lengths = rng.integers(100, 2000, 5)
    _run(cuda_device, rng, lengths, 2, 128, 8, bs, blocks_first, 0.4, True)


def test_batch_shared_partial_block_falls_back_in_order(cuda_device):
    rng = np.random.default_rng(9)
    lengths = [640, 1000, 300]
    _run(cuda_device, rng, lengths, 4, 256, 8, 16, False, 0.0, True, partial_conflict=True)


@pytest.mark.parametrize("dedup", [False, True])
def test_batch_interior_shared_block(cuda_device, dedup):
    rng = np.random.default_rng(17)
    _run(cuda_device, rng, [800, 500, 333], 4, 256, 8, 16, False, 0.0, dedup,
         interior_share=True)


def test_batch_fp8_sized_rows(cuda_device):
    rng = np.random.default_rng(12)
    _run(cuda_device, rng, [2048] * 16, 8, 128, 8, 16, False, 0.0, False)


@pytest.mark.parametrize("dedup", [False, True])
def test_batch_mixed_load_policies(cuda_device, dedup):
    """8-bit requests in one launch, some with every lane run on a 128-byte
    line (T and the first restored token multiples of 128: non-temporal loads)
    and some off the lines (cached loads)."""
    rng = np.random.default_rng(77)
    _run(cuda_device, rng, [1024, 1088, 2048, 1040, 1536, 1152], 8, 256, 8, 16, False, 0.5,
         dedup)

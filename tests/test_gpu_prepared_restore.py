"""Prepared fused restore (native_gpu.PreparedRestore over
origami_restore_plan_create / _launch): one plan per request, launched for
several layers (each its own stream and destination cache), gives byte for
byte what unpack_to_kv_cache gives per layer and what the oracle's unpack +
scatter gives (bitpack_layout_cuda.cu:91-128, benchmark_utils.py:350-444),
for planner-order, reordered and partial chunk plans, aligned and ragged
token counts, sub-byte widths and both cache layouts; it refuses a cache of
another geometry and a closed plan, and an irregular plan takes the
two-step path."""
import numpy as np
import pytest
import torch

from oracle import oracle
from origami_amd.layout import kv_symbol_layout
from origami_amd.lossless import native_gpu
from origami_amd.lossless.chunking import plan_head_channel_chunks

pytestmark = pytest.mark.gpu


def _specs(kind, T, H, C, rng, target=1 << 14):
    specs = [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
              c.layout.channel_end, 0, 2 * T]
             for c in plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C,
                                               token_count=2 * T, bytes_per_symbol=1,
                                               min_bytes=target, target_bytes=target,
                                               max_bytes=target)]
    if kind == "planner":
        return specs
    specs = [specs[i] for i in rng.permutation(len(specs))]
    if kind == "reordered_partial":
        specs = specs[: max(1, len(specs) * 2 // 3)]
    if kind == "irregular":  # one chunk covers half the tokens: no fused restore
        hs, he, cs, ce, _, _ = specs[0]
        specs[0] = [hs, he, cs, ce, 0, T]
    return specs


@pytest.mark.parametrize("kind,T,bits,bs,blocks_first", [
    ("planner", 2048, 8, 16, False),
    ("planner", 2053, 8, 16, True),
    ("planner", 1536, 4, 32, False),
    ("reordered", 1000, 8, 16, False),
    ("reordered_partial", 777, 3, 8, True),
    ("planner", 4096, 5, 16, False),
    # b = 1, 2, 4 with T a multiple of 128 / b: the wide 16-byte-run restore
    ("planner", 2048, 1, 16, True),
    ("planner", 2048, 2, 24, False),
    ("reordered", 1024, 4, 8, False),
    # fewer tokens than one lane run
    ("planner", 7, 8, 16, False),
    ("reordered", 15, 3, 8, True),
])
def test_prepared_restore_matches_fused_and_oracle(cuda_device, kind, T, bits, bs,
                                                   blocks_first):
    dev, H, C, layers = cuda_device, 4, 128, 3
    rng = np.random.default_rng(T * 10 + bits)
    specs = _specs(kind, T, H, C, rng)
    lay = kv_symbol_layout(T, H, C, bits, specs)
    nblk = -(-T // bs)
    NB = nblk + 9
    ids_np = rng.permutation(NB)[:nblk].astype(np.int64)
    shape = (NB, 2, bs, H, C // 2) if blocks_first else (2, NB, bs, H, C // 2)
    caches = [torch.full(shape, 7, dtype=torch.bfloat16, device=dev) for _ in range(layers)]
    prep = native_gpu.PreparedRestore(lay, T, caches[0], ids_np)
    assert prep.supported
    ids = native_gpu.block_ids_tensor(ids_np, dev, NB)
    for layer in range(layers):
        sym = rng.integers(0, 256, 2 * T * H * C, dtype=np.uint8)
        flat_np, offs = oracle.pack_canonical(sym, bits, specs, [2 * T, H, C], [0, 1, 2, -1])
        flat = torch.from_numpy(flat_np).to(dev)
        prep.restore(flat, caches[layer])
        ref = torch.full(shape, 7, dtype=torch.bfloat16, device=dev)
        native_gpu.unpack_to_kv_cache(flat, lay, T, ref, ids)
        got = caches[layer].view(torch.uint8).cpu().numpy()
        assert np.array_equal(got, ref.view(torch.uint8).cpu().numpy()), layer
        expect = torch.full(shape, 7, dtype=torch.bfloat16).view(torch.uint8).numpy().copy()
        oracle.restore_layer(flat_np, offs, bits, specs, T, H, C, ids_np, expect,
                             blocks_first=blocks_first)
        assert np.array_equal(got, expect), layer
    prep.close()


def test_prepared_restore_refuses_other_geometry_and_closed_plan(cuda_device):
    dev, T, H, C = cuda_device, 512, 2, 128
    rng = np.random.default_rng(5)
    specs = _specs("planner", T, H, C, rng)
    lay = kv_symbol_layout(T, H, C, 8, specs)
    cache = torch.zeros((2, 40, 16, H, C // 2), dtype=torch.bfloat16, device=dev)
    prep = native_gpu.PreparedRestore(lay, T, cache, np.arange(32))
    flat = torch.zeros(lay.stream_bytes, dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError, match="geometry differs"):
        prep.restore(flat, torch.zeros((2, 41, 16, H, C // 2), dtype=torch.bfloat16, device=dev))
    with pytest.raises(RuntimeError, match="geometry differs"):
        prep.restore(flat, cache.view(torch.float16))
    with pytest.raises(RuntimeError, match="exceed flat_chunks length"):
        prep.restore(flat[:-1], cache)
    prep.restore(flat, cache)
    prep.close()
    with pytest.raises(RuntimeError, match="closed"):
        prep.restore(flat, cache)


def test_prepared_restore_irregular_plan_takes_two_step_path(cuda_device):
    dev, T, H, C = cuda_device, 300, 2, 64
    rng = np.random.default_rng(6)
    specs = _specs("irregular", T, H, C, rng)
    lay = kv_symbol_layout(T, H, C, 8, specs)
    nblk = -(-T // 16)
    ids_np = rng.permutation(nblk + 3)[:nblk].astype(np.int64)
    cache = torch.zeros((2, nblk + 3, 16, H, C), dtype=torch.uint8, device=dev)
    prep = native_gpu.PreparedRestore(lay, T, cache, ids_np)
    assert not prep.supported
    sym = rng.integers(0, 256, 2 * T * H * C, dtype=np.uint8)
    flat_np, offs = oracle.pack_canonical(sym, 8, specs, [2 * T, H, C], [0, 1, 2, -1])
    prep.restore(torch.from_numpy(flat_np).to(dev), cache)
    expect = np.zeros(cache.shape, dtype=np.uint8)
    oracle.restore_layer(flat_np, offs, 8, specs, T, H, C, ids_np, expect)
    assert np.array_equal(cache.cpu().numpy(), expect)

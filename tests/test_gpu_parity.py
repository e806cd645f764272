"""Parity of the HIP layout path (liborigami_layout.so) with the CPU oracle.

Every comparison is bit-exact (integer/byte work).  Cases cover bits 1..8,
five source layouts, regular (planner) and irregular (token-split, partial)
chunk plans, both paged-cache layouts, ragged token counts, unaligned stream
pointers, and one full Llama-3-8B layer (32768 tokens) compared whole.
"""
import numpy as np
import pytest
import torch

from oracle import oracle
from origami_amd.layout import CanonicalLayout, kv_symbol_layout
from origami_amd import _native
from origami_amd.lossless import native_cpu, native_gpu
from origami_amd.lossless.chunking import plan_head_channel_chunks
from tests import bitref

pytestmark = pytest.mark.gpu

LAYOUTS = [
    (["token", "head", "head_dim"], [0, 1, 2, -1]),
    (["head", "token", "head_dim"], [1, 0, 2, -1]),
    (["head", "head_dim", "token"], [2, 0, 1, -1]),
    (["layer", "token", "head", "head_dim"], [1, 2, 3, 0]),
    (["token", "layer", "head_dim", "head"], [0, 3, 2, 1]),
]


def _shape(layout, T, H, C):
    return [{"token": T, "head": H, "head_dim": C, "layer": 1}[a] for a in layout]


def planner_specs(T, H, C, target):
    return np.asarray([[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
                        c.layout.channel_end, c.layout.token_start, c.layout.token_end]
                       for c in plan_head_channel_chunks(
                           layer_index=0, num_heads=H, head_dim=C, token_count=T,
                           bytes_per_symbol=1, min_bytes=target, target_bytes=target,
                           max_bytes=target)], dtype=np.int64)


def _gpu_u8(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _case_specs(kind, rng, T, H, C):
    if kind == "planner":
        return planner_specs(T, H, C, max(64, T * C // 3))
    if kind == "reversed":  # planner boxes stored in reverse order: regular, not dense
        return planner_specs(T, H, C, max(64, T * C // 3))[::-1].copy()
    if kind == "partition":
        return bitref.random_specs(rng, T, H, C, partition=True)
    if kind == "partial":  # a single box: the rest of the tensor is uncovered
        return np.asarray([[0, H, C // 4, C, 0, T]], np.int64)
    raise AssertionError(kind)


@pytest.mark.parametrize("kind", ["planner", "reversed", "partition", "partial"])
@pytest.mark.parametrize("bits", range(1, 9))
@pytest.mark.parametrize("li", range(len(LAYOUTS)))
def test_unpack_and_pack_match_oracle(cuda_device, li, bits, kind):
    layout, axes = LAYOUTS[li]
    rng = np.random.default_rng(1000 * li + 10 * bits + len(kind))
    for T, H, C in [(40, 2, 32), (257, 3, 48), (96, 1, 16)]:
        shape = _shape(layout, T, H, C)
        specs = _case_specs(kind, rng, T, H, C)
        sym = rng.integers(0, 256, int(np.prod(shape)), dtype=np.uint8)
        ref_flat, offs = oracle.pack_canonical(sym, bits, specs, shape, axes)
        ref_sym = oracle.unpack_canonical(ref_flat, offs, bits, specs, shape, axes)

        flat_gpu, lay = native_gpu.pack_canonical_storage_flat(
            _gpu_u8(sym, cuda_device), bits, shape, layout, specs)
        assert np.array_equal(lay.offsets, offs)
        assert np.array_equal(flat_gpu.cpu().numpy(), ref_flat), (T, H, C)

        out = native_gpu.unpack_canonical_storage_chunks(
            _gpu_u8(ref_flat, cuda_device), bits, shape, layout, specs, device=cuda_device)
        assert np.array_equal(out.cpu().numpy(), ref_sym), (T, H, C)


@pytest.mark.parametrize("shift", [1, 2, 3, 5])
@pytest.mark.parametrize("bits", [8, 3])
def test_unaligned_stream_pointer(cuda_device, shift, bits):
    rng = np.random.default_rng(shift)
    T, H, C = 64, 2, 32
    specs = planner_specs(T, H, C, 1024)
    sym = rng.integers(0, 256, T * H * C, dtype=np.uint8)
    ref_flat, offs = oracle.pack_canonical(sym, bits, specs, [T, H, C], [0, 1, 2, -1])
    buf = torch.zeros(ref_flat.size + 16, dtype=torch.uint8, device=cuda_device)
    buf[shift:shift + ref_flat.size] = _gpu_u8(ref_flat, cuda_device)
    view = buf[shift:shift + ref_flat.size]
    lay = CanonicalLayout.make([T, H, C], ["token", "head", "head_dim"], bits, specs)
    out = native_gpu.unpack_layout(view, lay)
    assert np.array_equal(out.cpu().numpy(), sym & ((1 << bits) - 1))
    # pack into an unaligned destination; the bytes around it stay untouched
    buf2 = torch.full((ref_flat.size + 16,), 0xAB, dtype=torch.uint8, device=cuda_device)
    native_gpu.pack_layout(_gpu_u8(sym, cuda_device), lay, buf2[shift:shift + ref_flat.size])
    host = buf2.cpu().numpy()
    assert np.array_equal(host[shift:shift + ref_flat.size], ref_flat)
    assert (host[:shift] == 0xAB).all() and (host[shift + ref_flat.size:] == 0xAB).all()


def test_empty_chunk_list_gives_zeros(cuda_device):
    out = native_gpu.unpack_canonical_storage_chunks(
        [], 8, [5, 2, 3], ["token", "head", "head_dim"], [], device=cuda_device)
    assert out.numel() == 30 and int(out.sum()) == 0


def _kv_case(rng, tokens, H, C, bs, blocks_first, extra_blocks=5):
    nblk = -(-tokens // bs)
    NB = nblk + extra_blocks
    ids = rng.permutation(NB)[:nblk].astype(np.int64)
    shape = (NB, 2, bs, H, C) if blocks_first else (2, NB, bs, H, C)
    cache = rng.integers(0, 256, shape, dtype=np.uint8)
    return ids, cache


@pytest.mark.parametrize("blocks_first", [False, True])
@pytest.mark.parametrize("bits", [8, 4, 3, 1])
@pytest.mark.parametrize("tokens,H,C,bs", [
    (4096, 8, 256, 16),    # Llama-3-8B bf16 geometry, 4096 tokens
    (1000, 8, 256, 16),    # ragged: last block partially filled
    (777, 4, 256, 32),     # Qwen2.5-7B heads, ragged, larger blocks
    (2048, 8, 128, 16),    # fp8 head bytes
    (100, 2, 64, 8),       # blocks smaller than a lane's 16 tokens
])
def test_restore_to_kv_cache_matches_oracle(cuda_device, tokens, H, C, bs, blocks_first, bits):
    rng = np.random.default_rng(tokens + bits + 7 * bs)
    specs = planner_specs(2 * tokens, H, C, 1 << 16)
    value = rng.integers(0, 256, (2, tokens, H, C), dtype=np.uint8)
    sym = value.reshape(-1)
    flat, offs = oracle.pack_canonical(sym, bits, specs, [2 * tokens, H, C], [0, 1, 2, -1])
    ids, cache = _kv_case(rng, tokens, H, C, bs, blocks_first)
    expect = cache.copy()
    oracle.restore_layer(flat, offs, bits, specs, tokens, H, C, ids, expect, blocks_first)

    cache_gpu = _gpu_u8(cache, cuda_device)
    lay = kv_symbol_layout(tokens, H, C, bits, specs)
    ids_gpu = native_gpu.block_ids_tensor(ids, cuda_device, cache.shape[1 if not blocks_first else 0])
    native_gpu.unpack_to_kv_cache(_gpu_u8(flat, cuda_device), lay, tokens, cache_gpu, ids_gpu)
    assert np.array_equal(cache_gpu.cpu().numpy(), expect)


@pytest.mark.parametrize("blocks_first", [False, True])
@pytest.mark.parametrize("bits", [8, 7, 4, 3, 2, 1])
@pytest.mark.parametrize("tokens,H,C,bs", [
    (4096, 8, 256, 16), (1000, 8, 256, 16), (2048, 8, 128, 16), (100, 2, 64, 8),
])
def test_save_from_kv_cache_matches_oracle(cuda_device, tokens, H, C, bs, blocks_first, bits):
    rng = np.random.default_rng(tokens * 3 + bits)
    specs = planner_specs(2 * tokens, H, C, 1 << 16)
    ids, cache = _kv_case(rng, tokens, H, C, bs, blocks_first)
    nblk = ids.size
    gathered = oracle.gather_kv_cache(cache, ids, blocks_first).reshape(2, nblk * bs, H, C)
    sym = np.ascontiguousarray(gathered[:, :tokens]).reshape(-1)
    ref_flat, _ = oracle.pack_canonical(sym, bits, specs, [2 * tokens, H, C], [0, 1, 2, -1])

    lay = kv_symbol_layout(tokens, H, C, bits, specs)
    cache_gpu = _gpu_u8(cache, cuda_device)
    ids_gpu = native_gpu.block_ids_tensor(ids, cuda_device)
    flat = native_gpu.pack_from_kv_cache(cache_gpu, ids_gpu, tokens, lay)
    assert np.array_equal(flat.cpu().numpy(), ref_flat)


@pytest.mark.parametrize("blocks_first", [False, True])
@pytest.mark.parametrize("bits", [8, 5, 3, 1])
@pytest.mark.parametrize("tokens,bs", [(1, 16), (2, 8), (7, 16), (15, 16), (17, 8)])
def test_tiny_token_counts_restore_and_save(cuda_device, tokens, bs, blocks_first, bits):
    """Token counts below or just past one lane's 16-token run: every lane
    run is the partial last one of its half, planes are a few bytes long
    (chunks of 16 bytes), and the stream ends inside most runs.  The restore
    into a cache of random bytes and the save from it both equal the oracle."""
    H, C = 2, 32
    rng = np.random.default_rng(tokens * 11 + bits + bs)
    specs = planner_specs(2 * tokens, H, C, 16)
    value = rng.integers(0, 256, (2, tokens, H, C), dtype=np.uint8)
    flat, offs = oracle.pack_canonical(value.reshape(-1), bits, specs, [2 * tokens, H, C],
                                       [0, 1, 2, -1])
    ids, cache = _kv_case(rng, tokens, H, C, bs, blocks_first)
    expect = cache.copy()
    oracle.restore_layer(flat, offs, bits, specs, tokens, H, C, ids, expect, blocks_first)
    lay = kv_symbol_layout(tokens, H, C, bits, specs)
    nb = cache.shape[0 if blocks_first else 1]
    cache_gpu = _gpu_u8(cache, cuda_device)
    ids_gpu = native_gpu.block_ids_tensor(ids, cuda_device, nb)
    native_gpu.unpack_to_kv_cache(_gpu_u8(flat, cuda_device), lay, tokens, cache_gpu, ids_gpu)
    assert np.array_equal(cache_gpu.cpu().numpy(), expect), "restore"

    gathered = oracle.gather_kv_cache(cache, ids, blocks_first).reshape(2, ids.size * bs, H, C)
    sym = np.ascontiguousarray(gathered[:, :tokens]).reshape(-1)
    ref, _ = oracle.pack_canonical(sym, bits, specs, [2 * tokens, H, C], [0, 1, 2, -1])
    packed = native_gpu.pack_from_kv_cache(_gpu_u8(cache, cuda_device), ids_gpu, tokens, lay)
    assert np.array_equal(packed.cpu().numpy(), ref), "save"


@pytest.mark.parametrize("blocks_first", [False, True])
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("tokens", [16384, 8192])
def test_smaller_workgroups_restore_and_save(cuda_device, tokens, bits, blocks_first):
    """Launches with fewer than two 16-wave tiles per CU run 8- or 4-wave
    workgroups (2048-byte rows: 16384 tokens -> 8 waves, 8192 -> 4 waves on
    a 256-CU device)."""
    rng = np.random.default_rng(tokens + bits)
    H, C, bs = 8, 256, 16
    specs = planner_specs(2 * tokens, H, C, 1 << 20)
    value = rng.integers(0, 256, (2, tokens, H, C), dtype=np.uint8)
    flat, offs = oracle.pack_canonical(value.reshape(-1), bits, specs, [2 * tokens, H, C],
                                       [0, 1, 2, -1])
    ids, cache = _kv_case(rng, tokens, H, C, bs, blocks_first)
    expect = cache.copy()
    oracle.restore_layer(flat, offs, bits, specs, tokens, H, C, ids, expect, blocks_first)
    cache_gpu = _gpu_u8(cache, cuda_device)
    lay = kv_symbol_layout(tokens, H, C, bits, specs)
    ids_gpu = native_gpu.block_ids_tensor(ids, cuda_device)
    native_gpu.unpack_to_kv_cache(_gpu_u8(flat, cuda_device), lay, tokens, cache_gpu, ids_gpu)
    assert np.array_equal(cache_gpu.cpu().numpy(), expect)
    back = native_gpu.pack_from_kv_cache(cache_gpu, ids_gpu, tokens, lay)
    assert np.array_equal(back.cpu().numpy(), flat)


@pytest.mark.parametrize("bits", [8, 5])
def test_non_dense_plan_restore_and_save(cuda_device, bits):
    """Planner boxes in reverse order: every plane still spans all tokens at
    one width, so the row kernels run, reading plane offsets from the
    uploaded plane table instead of the dense closed form."""
    rng = np.random.default_rng(40 + bits)
    tokens, H, C, bs = 1000, 4, 128, 16
    specs = planner_specs(2 * tokens, H, C, 1 << 15)[::-1].copy()
    assert len(specs) > 2
    value = rng.integers(0, 256, (2, tokens, H, C), dtype=np.uint8)
    flat, offs = oracle.pack_canonical(value.reshape(-1), bits, specs, [2 * tokens, H, C],
                                       [0, 1, 2, -1])
    ids, cache = _kv_case(rng, tokens, H, C, bs, False)
    expect = cache.copy()
    oracle.restore_layer(flat, offs, bits, specs, tokens, H, C, ids, expect, False)
    cache_gpu = _gpu_u8(cache, cuda_device)
    lay = kv_symbol_layout(tokens, H, C, bits, specs)
    ids_gpu = native_gpu.block_ids_tensor(ids, cuda_device)
    flat_gpu = _gpu_u8(flat, cuda_device)
    code, nb, bsz, heads, hb = native_gpu.cache_geometry(cache_gpu)
    stream = native_gpu._stream_handle(cuda_device)
    # called directly: the fused entry points must accept this plan (the
    # Python wrappers would fall back silently)
    _native.call("origami_unpack_canonical_to_kv_cache", flat_gpu.data_ptr(), flat_gpu.numel(),
                 *native_gpu._layout_args(lay), tokens, cache_gpu.data_ptr(), code, nb, bsz,
                 heads, hb, ids_gpu.data_ptr(), ids_gpu.numel(), stream)
    assert np.array_equal(cache_gpu.cpu().numpy(), expect)
    back = torch.empty_like(flat_gpu)
    _native.call("origami_pack_canonical_from_kv_cache", cache_gpu.data_ptr(), code, nb, bsz,
                 heads, hb, ids_gpu.data_ptr(), ids_gpu.numel(), tokens,
                 *native_gpu._layout_args(lay), back.data_ptr(), back.numel(), stream)
    assert np.array_equal(back.cpu().numpy(), flat)


@pytest.mark.parametrize("bits", [1, 2, 3, 5, 6, 7])
@pytest.mark.parametrize("shift", [0, 2, 1])
def test_lane_runs_at_the_stream_end(cuda_device, bits, shift):
    """Chunks covering 5 or 11 channels of one head: the stream ends 2 bytes
    past a dword boundary for odd widths, so the last lane runs cannot use
    the whole-dword window and take the guarded loads.  A nonzero `shift`
    moves the stream pointer off dword alignment (guarded addressing)."""
    rng = np.random.default_rng(bits * 10 + shift)
    for T, specs in [(16, [[0, 1, 0, 5, 0, 16]]), (48, [[0, 1, 3, 14, 0, 48]]),
                     (32, [[0, 1, 0, 5, 0, 32], [0, 1, 5, 16, 0, 32]])]:
        H, C = 1, 16
        specs = np.asarray(specs, np.int64)
        sym = rng.integers(0, 256, T * H * C, dtype=np.uint8)
        ref_flat, offs = oracle.pack_canonical(sym, bits, specs, [T, H, C], [0, 1, 2, -1])
        ref_sym = oracle.unpack_canonical(ref_flat, offs, bits, specs, [T, H, C], [0, 1, 2, -1])
        lay = CanonicalLayout.make([T, H, C], ["token", "head", "head_dim"], bits, specs)
        buf = torch.zeros(ref_flat.size + 8, dtype=torch.uint8, device=cuda_device)
        view = buf[shift:shift + ref_flat.size]
        view.copy_(_gpu_u8(ref_flat, cuda_device))
        out = native_gpu.unpack_layout(view, lay)
        assert np.array_equal(out.cpu().numpy(), ref_sym), (T, specs.tolist())
        buf2 = torch.full((ref_flat.size + 8,), 0xAB, dtype=torch.uint8, device=cuda_device)
        native_gpu.pack_layout(_gpu_u8(sym, cuda_device), lay, buf2[shift:shift + ref_flat.size])
        host = buf2.cpu().numpy()
        assert np.array_equal(host[shift:shift + ref_flat.size], ref_flat), (T, specs.tolist())
        assert (host[:shift] == 0xAB).all() and (host[shift + ref_flat.size:] == 0xAB).all()


def test_plan_cache_eviction_keeps_results(cuda_device):
    """300 distinct non-dense layouts (each uploads its plane table; the
    cache drops every plan after 256 uploads) interleaved with dense ones,
    each unpacked and checked; the first layout is used again at the end."""
    rng = np.random.default_rng(77)
    H, C, bits = 1, 32, 8
    cases = []
    for k in range(300):
        T = 16 * (k + 1)
        reordered = np.asarray([[0, 1, 16, 32, 0, T], [0, 1, 0, 16, 0, T]], np.int64)
        cases.append((T, reordered))
        if k % 5 == 0:
            cases.append((T, reordered[::-1].copy()))  # dense order
    cases.append(cases[1])
    for T, specs in cases:
        sym = rng.integers(0, 256, T * H * C, dtype=np.uint8)
        ref_flat, offs = oracle.pack_canonical(sym, bits, specs, [T, H, C], [0, 1, 2, -1])
        lay = CanonicalLayout.make([T, H, C], ["token", "head", "head_dim"], bits, specs)
        out = native_gpu.unpack_layout(_gpu_u8(ref_flat, cuda_device), lay)
        assert np.array_equal(out.cpu().numpy(), sym), (T, specs.tolist())
        flat = native_gpu.pack_layout(_gpu_u8(sym, cuda_device), lay)
        assert np.array_equal(flat.cpu().numpy(), ref_flat), (T, specs.tolist())


def test_concurrent_restores_from_threads(cuda_device):
    """Four threads, each on its own stream, restore and re-pack layers with
    dense and reordered plans (plans created and uploaded concurrently)."""
    import threading

    errors = []

    def worker(tid):
        try:
            rng = np.random.default_rng(900 + tid)
            stream = torch.cuda.Stream(device=cuda_device)
            with torch.cuda.stream(stream):
                for it in range(12):
                    tokens = 16 * int(rng.integers(4, 40)) + (it % 2) * 5
                    H, C, bs = 2, 64, 16
                    specs = planner_specs(2 * tokens, H, C, 1 << 12)
                    if (tid + it) % 2:
                        specs = specs[::-1].copy()
                    value = rng.integers(0, 256, (2, tokens, H, C), dtype=np.uint8)
                    flat, offs = oracle.pack_canonical(value.reshape(-1), 8, specs,
                                                       [2 * tokens, H, C], [0, 1, 2, -1])
                    ids, cache = _kv_case(rng, tokens, H, C, bs, bool(it % 3 == 0))
                    expect = cache.copy()
                    oracle.restore_layer(flat, offs, 8, specs, tokens, H, C, ids, expect,
                                         bool(it % 3 == 0))
                    cache_gpu = _gpu_u8(cache, cuda_device)
                    lay = kv_symbol_layout(tokens, H, C, 8, specs)
                    ids_gpu = native_gpu.block_ids_tensor(ids, cuda_device)
                    native_gpu.unpack_to_kv_cache(_gpu_u8(flat, cuda_device), lay, tokens,
                                                  cache_gpu, ids_gpu)
                    back = native_gpu.pack_from_kv_cache(cache_gpu, ids_gpu, tokens, lay)
                    stream.synchronize()
                    if not np.array_equal(cache_gpu.cpu().numpy(), expect):
                        errors.append((tid, it, "restore"))
                    if not np.array_equal(back.cpu().numpy(), flat):
                        errors.append((tid, it, "save"))
        except Exception as exc:  # noqa: BLE001 - reported below
            errors.append((tid, repr(exc)))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors


def test_irregular_plan_restore_falls_back_and_matches(cuda_device):
    rng = np.random.default_rng(5)
    tokens, H, C, bs = 300, 2, 32, 16
    specs = bitref.random_specs(rng, 2 * tokens, H, C, partition=True)  # token-split boxes
    value = rng.integers(0, 256, (2, tokens, H, C), dtype=np.uint8)
    flat, offs = oracle.pack_canonical(value.reshape(-1), 6, specs, [2 * tokens, H, C],
                                       [0, 1, 2, -1])
    ids, cache = _kv_case(rng, tokens, H, C, bs, False)
    expect = cache.copy()
    oracle.restore_layer(flat, offs, 6, specs, tokens, H, C, ids, expect, False)
    cache_gpu = _gpu_u8(cache, cuda_device)
    lay = kv_symbol_layout(tokens, H, C, 6, specs)
    native_gpu.unpack_to_kv_cache(_gpu_u8(flat, cuda_device), lay, tokens, cache_gpu,
                                  native_gpu.block_ids_tensor(ids, cuda_device))
    assert np.array_equal(cache_gpu.cpu().numpy(), expect)


@pytest.mark.parametrize("tokens,H,C,bs", [
    (1234, 8, 256, 16),   # 32 KiB block-halves, partial last block
    (1000, 4, 512, 40),   # 80 KiB block-halves: three unrolled rounds per workgroup
    (77, 2, 48, 24),      # 96-byte rows
    (300, 3, 20, 8),      # 60-byte rows: the byte path
])
@pytest.mark.parametrize("blocks_first", [False, True])
def test_block_scatter_and_gather_match_oracle(cuda_device, blocks_first, tokens, H, C, bs):
    rng = np.random.default_rng(11 + tokens)
    value = rng.integers(0, 256, (2, tokens, H, C), dtype=np.uint8)
    ids, cache = _kv_case(rng, tokens, H, C, bs, blocks_first)
    expect = cache.copy()
    oracle.scatter_kv_cache(value, tokens, H, C, ids, expect, blocks_first)
    cache_gpu = _gpu_u8(cache, cuda_device)
    ids_gpu = native_gpu.block_ids_tensor(ids, cuda_device)
    native_gpu.scatter_kv_blocks(_gpu_u8(value, cuda_device), tokens, cache_gpu, ids_gpu)
    assert np.array_equal(cache_gpu.cpu().numpy(), expect)
    back = native_gpu.gather_kv_blocks(cache_gpu, ids_gpu)
    assert np.array_equal(back.cpu().numpy(), oracle.gather_kv_cache(expect, ids, blocks_first))


def test_typed_bf16_cache_round_trip(cuda_device):
    """bf16 cache tensors (not uint8 views) go through the same byte path."""
    torch.manual_seed(0)
    tokens, H, D, bs = 512, 8, 128, 16
    nblk = tokens // bs
    kv = torch.randn(2, nblk, bs, H, D, dtype=torch.bfloat16, device=cuda_device)
    ids = torch.randperm(nblk + 3)[:nblk]
    cache = torch.zeros(2, nblk + 3, bs, H, D, dtype=torch.bfloat16, device=cuda_device)
    cache[:, ids.to(cuda_device)] = kv
    specs = planner_specs(2 * tokens, H, 2 * D, 1 << 16)
    lay = kv_symbol_layout(tokens, H, 2 * D, 8, specs)
    ids_gpu = native_gpu.block_ids_tensor(ids, cuda_device)
    flat = native_gpu.pack_from_kv_cache(cache, ids_gpu, tokens, lay)
    # the stream is the byte-plane transpose of the token-major K/V bytes
    sym = kv.reshape(2 * tokens, H, D).contiguous().view(torch.uint8).cpu().numpy()
    ref, _ = oracle.pack_canonical(sym.reshape(-1), 8, specs, [2 * tokens, H, 2 * D],
                                   [0, 1, 2, -1])
    assert np.array_equal(flat.cpu().numpy(), ref)
    cache2 = torch.zeros_like(cache)
    native_gpu.unpack_to_kv_cache(flat, lay, tokens, cache2, ids_gpu)
    assert torch.equal(cache2.view(torch.int16), cache.view(torch.int16))


def test_full_llama3_8b_layer_matches_oracle(cuda_device):
    """One full Llama-3-8B layer: 32768 tokens, 8 KV heads, bf16 (128 MiB of
    K/V), 1 MiB chunks, randomly permuted block table; pack and restore are
    compared whole with the oracle."""
    tokens, H, C, bs = 32768, 8, 256, 16
    rng = np.random.default_rng(1)
    specs = planner_specs(2 * tokens, H, C, 1 << 20)
    assert specs.shape[0] == 128
    nblk = tokens // bs
    NB = nblk + 64
    ids = rng.permutation(NB)[:nblk].astype(np.int64)
    cache = torch.randint(0, 256, (2, NB, bs, H, C), dtype=torch.uint8, device=cuda_device)
    cache_np = cache.cpu().numpy()
    lay = kv_symbol_layout(tokens, H, C, 8, specs)
    ids_gpu = native_gpu.block_ids_tensor(ids, cuda_device)
    flat = native_gpu.pack_from_kv_cache(cache, ids_gpu, tokens, lay)
    sym = oracle.gather_kv_cache(cache_np, ids)
    ref_flat, offs = oracle.pack_canonical(sym, 8, specs, [2 * tokens, H, C], [0, 1, 2, -1])
    assert np.array_equal(flat.cpu().numpy(), ref_flat)

    ids2 = rng.permutation(NB)[:nblk].astype(np.int64)
    dst = torch.randint(0, 256, (2, NB, bs, H, C), dtype=torch.uint8, device=cuda_device)
    expect = dst.cpu().numpy()
    oracle.restore_layer(ref_flat, offs, 8, specs, tokens, H, C, ids2, expect)
    native_gpu.unpack_to_kv_cache(flat, lay, tokens, dst, native_gpu.block_ids_tensor(ids2, cuda_device))
    assert np.array_equal(dst.cpu().numpy(), expect)


def test_native_cpu_api_round_trip(cuda_device):
    """native_cpu.pack/unpack_canonical_storage_chunks: the reference's stubs,
    working here through the GPU and returning CPU tensors."""
    rng = np.random.default_rng(9)
    T, H, C = 200, 2, 32
    specs = planner_specs(T, H, C, 2048).tolist()
    sym = torch.from_numpy(rng.integers(0, 16, T * H * C, dtype=np.uint8))
    chunks = native_cpu.pack_canonical_storage_chunks(sym, 4, [T, H, C],
                                                      ["token", "head", "head_dim"], specs)
    assert all(c.device.type == "cpu" for c in chunks)
    ref_flat, offs = oracle.pack_canonical(sym.numpy(), 4, specs, [T, H, C], [0, 1, 2, -1])
    assert [c.numel() for c in chunks] == np.diff(offs).tolist()
    assert np.array_equal(torch.cat(chunks).numpy(), ref_flat)
    back = native_cpu.unpack_head_channel_chunks(chunks, 4, T, H, C, specs)
    assert back.device.type == "cpu" and torch.equal(back, sym)


def test_reference_extension_surface(cuda_device):
    """unpack_canonical_storage_chunks_cuda with the reference's argument list
    (bitpack_layout_cuda.cpp:316-325)."""
    rng = np.random.default_rng(4)
    T, H, C = 64, 2, 16
    specs = planner_specs(T, H, C, 512)
    sym = rng.integers(0, 32, T * H * C, dtype=np.uint8)
    flat, offs = oracle.pack_canonical(sym, 5, specs, [T, H, C], [0, 1, 2, -1])
    ext = native_gpu.load_bitpack_cuda_extension()
    out = ext.unpack_canonical_storage_chunks_cuda(
        _gpu_u8(flat, cuda_device), torch.from_numpy(offs).to(cuda_device),
        torch.full((specs.shape[0],), 5, dtype=torch.int64, device=cuda_device),
        torch.tensor([T, H, C]), torch.tensor([0, 1, 2, -1]), T, H, C,
        torch.from_numpy(specs).to(cuda_device))
    assert np.array_equal(out.cpu().numpy(), sym)
    with pytest.raises(RuntimeError, match="byte size mismatch"):
        bad = offs.copy()
        bad[1:] += 1
        ext.unpack_canonical_storage_chunks_cuda(
            _gpu_u8(np.zeros(bad[-1], np.uint8), cuda_device), torch.from_numpy(bad),
            torch.full((specs.shape[0],), 5, dtype=torch.int64), torch.tensor([T, H, C]),
            torch.tensor([0, 1, 2, -1]), T, H, C, torch.from_numpy(specs))


def test_errors_raise_with_reference_messages(cuda_device):
    with pytest.raises(RuntimeError, match="1..8 bit"):
        native_gpu.unpack_canonical_storage_chunks(
            [torch.zeros(8, dtype=torch.uint8)], 9, [8, 1, 1], ["token", "head", "head_dim"],
            [[0, 1, 0, 1, 0, 8]], device=cuda_device)
    cache = torch.zeros(2, 4, 16, 1, 16, dtype=torch.uint8, device=cuda_device)
    with pytest.raises(RuntimeError, match="block id out of range"):
        native_gpu.block_ids_tensor([4], cuda_device, 4)
    lay = kv_symbol_layout(100, 1, 16, 8, [[0, 1, 0, 16, 0, 200]])
    with pytest.raises(RuntimeError, match="tokens exceed destination block capacity"):
        native_gpu.unpack_to_kv_cache(torch.zeros(3200, dtype=torch.uint8, device=cuda_device),
                                      lay, 100, cache,
                                      native_gpu.block_ids_tensor([0, 1], cuda_device))

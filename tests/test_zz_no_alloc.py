"""Allocation-free fused restore: origami_unpack_canonical_to_kv_cache_noalloc,
called through the C ABI, gives byte for byte what
origami_unpack_canonical_to_kv_cache gives, on two calls in a row (the
second with a smaller layer), for chunk plans in the planner's order (no
device metadata) and reordered ones (plane table in the fixed scratch
array, rewritten by every call), at b = 8, 5 and in the wide 16-byte-run
mode (b = 4, 2); it creates no plan and makes no device allocation; it can
be captured in a HIP graph whose replays restore new stream contents; it
refuses a reordered-plan call from a second stream while the first
stream's call is still pending; and it rejects a reordered plan above the
scratch maximum."""
import numpy as np
import pytest
import torch

from oracle import oracle
from origami_amd import _native
from origami_amd.layout import kv_symbol_layout
from origami_amd.lossless import native_gpu
from origami_amd.lossless.chunking import plan_head_channel_chunks

pytestmark = pytest.mark.gpu

FUSED = "origami_unpack_canonical_to_kv_cache"
NOALLOC = "origami_unpack_canonical_to_kv_cache_noalloc"


def _planner_specs(T2, H, C, target):
    return [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
             c.layout.channel_end, 0, T2]
            for c in plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C,
                                              token_count=T2, bytes_per_symbol=1,
                                              min_bytes=target, target_bytes=target,
                                              max_bytes=target)]


def _specs(kind, T, H, C, rng):
    specs = _planner_specs(2 * T, H, C, 1 << 14)
    if kind == "planner":
        return specs
    order = rng.permutation(len(specs))
    specs = [specs[i] for i in order]
    if kind == "reordered_partial":
        specs = specs[: max(1, len(specs) * 2 // 3)]  # some planes uncovered -> zeros
    return specs


def _restore(name, flat, lay, T, cache, ids):
    code, nb, bs, H, C = native_gpu.cache_geometry(cache)
    _native.call(name, flat.data_ptr(), flat.numel(), *lay.native_args, int(T),
                 cache.data_ptr(), code, nb, bs, H, C, ids.data_ptr(), ids.numel(),
                 native_gpu._stream_handle(cache.device))


def _case(dev, rng, kind, T, H, C, bits, bs, blocks_first):
    nblk = -(-T // bs)
    NB = nblk + 11
    specs = _specs(kind, T, H, C, rng)
    lay = kv_symbol_layout(T, H, C, bits, specs)
    sym = rng.integers(0, 256, 2 * T * H * C, dtype=np.uint8)
    flat_np, offs = oracle.pack_canonical(sym, bits, specs, [2 * T, H, C], [0, 1, 2, -1])
    flat = torch.from_numpy(flat_np).to(dev)
    ids_np = rng.permutation(NB)[:nblk].astype(np.int64)
    ids = torch.from_numpy(ids_np).to(dev)
    shape = (NB, 2, bs, H, C) if blocks_first else (2, NB, bs, H, C)
    caches = {name: torch.full(shape, 0x5A, dtype=torch.uint8, device=dev)
              for name in (FUSED, NOALLOC)}
    for name, cache in caches.items():
        _restore(name, flat, lay, T, cache, ids)
    torch.cuda.synchronize(dev)
    got = caches[NOALLOC].cpu().numpy()
    assert np.array_equal(got, caches[FUSED].cpu().numpy()), (kind, T, H, C, bits)
    expect = np.full(shape, 0x5A, dtype=np.uint8)
    oracle.restore_layer(flat_np, offs, bits, specs, T, H, C, ids_np, expect,
                         blocks_first=blocks_first)
    assert np.array_equal(got, expect), (kind, T, H, C, bits)


@pytest.mark.parametrize("kind", ["planner", "reordered", "reordered_partial"])
@pytest.mark.parametrize("bits", [8, 5])
def test_noalloc_matches_fused_restore_twice(cuda_device, kind, bits):
    rng = np.random.default_rng(100 + bits)
    # first call, then a smaller layer (fewer tokens, heads and channels),
    # then one of 7 tokens (a single partial lane run per half)
    _case(cuda_device, rng, kind, 1000, 8, 256, bits, 16, False)
    _case(cuda_device, rng, kind, 300, 4, 128, bits, 16, True)
    _case(cuda_device, rng, kind, 7, 2, 32, bits, 16, False)


def test_noalloc_alternating_plans_rewrite_scratch(cuda_device):
    """A reordered plan, then a partial one of the same geometry: planes the
    second plan leaves uncovered must read as uncovered, not as the first
    call's offsets still in the scratch array."""
    rng = np.random.default_rng(7)
    for kind in ("reordered", "reordered_partial", "reordered", "planner"):
        _case(cuda_device, rng, kind, 640, 4, 256, 8, 16, False)


def test_noalloc_rejects_reordered_plan_above_scratch_maximum(cuda_device):
    T, H, C, bs = 16, 1024, 256, 16  # 262144 planes > 131072
    specs = [[H // 2, H, 0, C, 0, 2 * T], [0, H // 2, 0, C, 0, 2 * T]]
    lay = kv_symbol_layout(T, H, C, 8, specs)
    flat = torch.zeros(lay.stream_bytes, dtype=torch.uint8, device=cuda_device)
    cache = torch.zeros((2, 2, bs, H, C), dtype=torch.uint8, device=cuda_device)
    ids = torch.tensor([1], dtype=torch.int64, device=cuda_device)
    with pytest.raises(_native.OrigamiNativeError, match="at most 131072") as err:
        _restore(NOALLOC, flat, lay, T, cache, ids)
    assert err.value.code == _native.ORIGAMI_ERR_UNSUPPORTED
    # the allocating entry point serves it (its plane table is allocated)
    _restore(FUSED, flat, lay, T, cache, ids)
    torch.cuda.synchronize(cuda_device)


@pytest.mark.parametrize("kind", ["planner", "reordered"])
def test_noalloc_wide_runs_twice(cuda_device, kind):
    """b = 4 then b = 2 (token counts multiples of 128 / b): the wide
    16-byte-run restore, second call smaller."""
    rng = np.random.default_rng(300)
    _case(cuda_device, rng, kind, 1024, 8, 256, 4, 16, False)
    _case(cuda_device, rng, kind, 512, 4, 128, 2, 16, True)


def test_noalloc_creates_no_plan_and_allocates_nothing(cuda_device):
    dev = cuda_device
    rng = np.random.default_rng(11)
    calls = []
    for kind, T, bits in (("planner", 700, 8), ("reordered", 700, 8),
                          ("reordered_partial", 512, 4), ("planner", 1024, 2)):
        H, C, bs = 4, 128, 16
        nblk = -(-T // bs)
        NB = nblk + 3
        specs = _specs(kind, T, H, C, rng)
        lay = kv_symbol_layout(T, H, C, bits, specs)
        flat = torch.from_numpy(rng.integers(0, 256, lay.stream_bytes, dtype=np.uint8)).to(dev)
        cache = torch.zeros((2, NB, bs, H, C), dtype=torch.uint8, device=dev)
        ids = torch.from_numpy(rng.permutation(NB)[:nblk].astype(np.int64)).to(dev)
        calls.append((flat, lay, T, cache, ids))
    before = _native.debug_counters()
    for _ in range(2):
        for c in calls:
            _restore(NOALLOC, *c)
    torch.cuda.synchronize(dev)
    assert _native.debug_counters() == before
    # the allocating entry point, on the same reordered plan, creates a plan
    # and uploads its plane table (the counters see both)
    _restore(FUSED, *calls[1])
    torch.cuda.synchronize(dev)
    after = _native.debug_counters()
    assert after[0] > before[0] and after[1] > before[1]


@pytest.mark.parametrize("kind,bits", [("planner", 8), ("reordered", 8), ("reordered", 3)])
def test_noalloc_graph_capture_replays(cuda_device, kind, bits):
    """The restore captured once (single stream, kernels only); each replay
    after new stream bytes are copied into the captured input restores
    them, checked against the allocating entry point and the oracle, with
    eager work and synchronisation between the replays."""
    dev = cuda_device
    rng = np.random.default_rng(400 + bits)
    T, H, C, bs = 1000, 8, 256, 16
    nblk = -(-T // bs)
    NB = nblk + 5
    specs = _specs(kind, T, H, C, rng)
    lay = kv_symbol_layout(T, H, C, bits, specs)
    ids_np = rng.permutation(NB)[:nblk].astype(np.int64)
    ids = torch.from_numpy(ids_np).to(dev)
    flat = torch.zeros(lay.stream_bytes, dtype=torch.uint8, device=dev)
    cache = torch.zeros((2, NB, bs, H, C), dtype=torch.uint8, device=dev)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        _restore(NOALLOC, flat, lay, T, cache, ids)  # warm-up outside the capture
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _restore(NOALLOC, flat, lay, T, cache, ids)
    for replay in range(3):
        sym = rng.integers(0, 256, 2 * T * H * C, dtype=np.uint8)
        flat_np, offs = oracle.pack_canonical(sym, bits, specs, [2 * T, H, C], [0, 1, 2, -1])
        flat.copy_(torch.from_numpy(flat_np).to(dev))
        cache.fill_(0x5A)
        torch.cuda.synchronize(dev)
        graph.replay()
        torch.cuda.synchronize(dev)
        ref = torch.full_like(cache, 0x5A)
        _restore(FUSED, flat, lay, T, ref, ids)
        torch.cuda.synchronize(dev)
        got = cache.cpu().numpy()
        assert np.array_equal(got, ref.cpu().numpy()), (kind, bits, replay)
        expect = np.full(cache.shape, 0x5A, dtype=np.uint8)
        oracle.restore_layer(flat_np, offs, bits, specs, T, H, C, ids_np, expect)
        assert np.array_equal(got, expect), (kind, bits, replay)
    del graph


def test_noalloc_refuses_overlapping_call_from_another_stream(cuda_device):
    """A reordered-plan call queued on stream A behind a long spin, then one
    on stream B before A has run: B's call is refused (the two would share
    the scratch plane table); after A completes, B's call runs and matches
    the oracle."""
    dev = cuda_device
    rng = np.random.default_rng(500)
    T, H, C, bs = 640, 4, 256, 16
    nblk = -(-T // bs)
    NB = nblk + 3
    specs = _specs("reordered", T, H, C, rng)
    lay = kv_symbol_layout(T, H, C, 8, specs)
    sym = rng.integers(0, 256, 2 * T * H * C, dtype=np.uint8)
    flat_np, offs = oracle.pack_canonical(sym, 8, specs, [2 * T, H, C], [0, 1, 2, -1])
    flat = torch.from_numpy(flat_np).to(dev)
    ids_np = rng.permutation(NB)[:nblk].astype(np.int64)
    ids = torch.from_numpy(ids_np).to(dev)
    caches = [torch.zeros((2, NB, bs, H, C), dtype=torch.uint8, device=dev) for _ in range(2)]
    sa, sb = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    torch.cuda.synchronize(dev)
    # a bounded spin of about 200 ms (calibrated with events) ahead of A's
    # restore, so A is still pending when B's call comes, whatever the host does
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    torch.cuda._sleep(1 << 22)
    end.record()
    end.synchronize()
    ms_per_cycle = max(start.elapsed_time(end), 1e-3) / (1 << 22)
    with torch.cuda.stream(sa):
        torch.cuda._sleep(int(min(200.0 / ms_per_cycle, 4e10)))
        _restore(NOALLOC, flat, lay, T, caches[0], ids)
    with torch.cuda.stream(sb):
        with pytest.raises(_native.OrigamiNativeError, match="must not overlap") as err:
            _restore(NOALLOC, flat, lay, T, caches[1], ids)
    assert err.value.code == _native.ORIGAMI_ERR_INVALID
    torch.cuda.synchronize(dev)
    with torch.cuda.stream(sb):
        _restore(NOALLOC, flat, lay, T, caches[1], ids)
    torch.cuda.synchronize(dev)
    expect = np.zeros(caches[0].shape, dtype=np.uint8)
    oracle.restore_layer(flat_np, offs, 8, specs, T, H, C, ids_np, expect)
    for c in caches:
        assert np.array_equal(c.cpu().numpy(), expect)

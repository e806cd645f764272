"""Chunk planner (lossless/chunking.py:22-123 of the reference), pinned by
hand-worked plans.  Counts for the benchmark geometries: one layer's K/V is
the symbol tensor [2T, H, D*e] with 1 MiB min/target/max chunks."""
import pytest

from origami_amd.lossless.chunking import plan_head_channel_chunks

MIB = 1 << 20


def plan(H, C, T, mn=MIB, tg=MIB, mx=MIB, bps=1):
    return plan_head_channel_chunks(layer_index=3, num_heads=H, head_dim=C, token_count=T,
                                    bytes_per_symbol=bps, min_bytes=mn, target_bytes=tg,
                                    max_bytes=mx)


def boxes(p):
    return [(c.layout.head_start, c.layout.head_end, c.layout.channel_start,
             c.layout.channel_end) for c in p]


@pytest.mark.parametrize("H,C,T2,count,width", [
    (8, 256, 2 * 4096, 16, 128),     # Llama-3-8B, 4096 tokens, bf16
    (8, 256, 2 * 32768, 128, 16),    # Llama-3-8B, 32768 tokens, bf16
    (8, 128, 2 * 16384, 32, 32),     # Llama-3-8B, 16384 tokens, fp8
    (8, 256, 2 * 131072, 512, 4),    # Llama-3-70B geometry, 131072 tokens
])
def test_benchmark_geometries(H, C, T2, count, width):
    p = plan(H, C, T2)
    assert len(p) == count
    assert all(c.layout.channel_end - c.layout.channel_start == width for c in p)
    assert all(c.layout.unpacked_bytes == MIB for c in p)
    assert [c.chunk_id for c in p] == list(range(count))
    assert all(c.layout.layer_index == 3 for c in p)


def test_ragged_channel_split():
    # 2T = 20000: 1 MiB // 20000 = 52 channels; 256 = 4*52 + 48
    p = plan(4, 256, 20000)
    assert len(p) == 20
    assert [c.layout.channel_end - c.layout.channel_start for c in p[:5]] == [52, 52, 52, 52, 48]
    assert boxes(p)[:5] == [(0, 1, 0, 52), (0, 1, 52, 104), (0, 1, 104, 156),
                           (0, 1, 156, 208), (0, 1, 208, 256)]


def test_small_heads_are_grouped():
    assert boxes(plan(8, 256, 64)) == [(0, 8, 0, 256)]
    # target 1000 B, min 1200 B, 10 tokens x 4 channels per head = 40 B:
    # start from 25 heads (1000 B), grow to 30 heads (1200 B); then the
    # remaining 10 heads form the last group.
    p = plan(40, 4, 10, mn=1200, tg=1000, mx=1000)
    assert boxes(p) == [(0, 30, 0, 4), (30, 40, 0, 4)]
    assert [c.layout.unpacked_bytes for c in p] == [1200, 400]


def test_min_width_raises_all_but_last_piece():
    # 100-byte channels: target 3, max 5, min 4 channels -> widths 4, 4, 2
    p = plan(1, 10, 100, mn=450, tg=300, mx=500)
    assert boxes(p) == [(0, 1, 0, 4), (0, 1, 4, 8), (0, 1, 8, 10)]


def test_last_single_head_is_one_chunk():
    # 10-byte channels, target 100 B = 10 channels = 2 whole heads per group;
    # the last head is alone, so it takes the channel path as one piece
    assert boxes(plan(3, 4, 10, mn=10, tg=100, mx=100)) == [(0, 2, 0, 4), (2, 3, 0, 4)]
    # one head only: channel path, one piece
    assert boxes(plan(1, 4, 10, mn=10, tg=100, mx=100)) == [(0, 1, 0, 4)]


def test_bytes_per_symbol_scales_channel_bytes():
    p = plan(2, 8, 1000, mn=4000, tg=4000, mx=4000, bps=2)
    assert [c.layout.channel_end - c.layout.channel_start for c in p] == [2, 2, 2, 2] * 2
    assert all(c.layout.unpacked_bytes == 4000 for c in p)


@pytest.mark.parametrize("H,C,T", [(8, 256, 8192), (4, 256, 2 * 12345), (3, 100, 777),
                                   (16, 64, 50)])
def test_plan_tiles_every_plane_once(H, C, T):
    seen = [[0] * C for _ in range(H)]
    for c in plan(H, C, T):
        L = c.layout
        assert (L.token_start, L.token_end) == (0, T)
        for h in range(L.head_start, L.head_end):
            for ch in range(L.channel_start, L.channel_end):
                seen[h][ch] += 1
    assert all(v == 1 for row in seen for v in row)


def test_empty_inputs():
    assert plan(0, 4, 4) == [] and plan(2, 0, 4) == [] and plan(2, 4, 0) == []

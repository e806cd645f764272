"""Chunk planner: cuts one layer's symbol tensor into ~target-size boxes.

Behaviour follows plan_head_channel_chunks (lossless/chunking.py:22-123 of the
reference) exactly, because the plan fixes the stream order and the chunk
boundaries of the wire format:

* a "channel" holds token_count * bytes_per_symbol bytes;
* when a whole head is smaller than target_bytes and more than one head
  remains, whole heads are grouped (as many as fit target and max, at least
  one, then grown until the group reaches min_bytes);
* otherwise the head is split along channels into widths
  min(remaining, target, max) channels, raised to min_bytes worth of channels
  unless it is the head's last piece.
"""
from __future__ import annotations

from dataclasses import dataclass

from origami_amd.metadata import ChunkLayout


@dataclass(frozen=True)
class PlannedChunk:
    chunk_id: int
    layout: ChunkLayout


def _box_bytes(tokens: int, channels: int, bytes_per_symbol: int) -> int:
    return max(0, int(tokens)) * max(0, int(channels)) * max(1, int(bytes_per_symbol))


def plan_head_channel_chunks(
    *,
    layer_index: int,
    num_heads: int,
    head_dim: int,
    token_count: int,
    bytes_per_symbol: int,
    min_bytes: int,
    target_bytes: int,
    max_bytes: int,
) -> list[PlannedChunk]:
    if num_heads <= 0 or head_dim <= 0 or token_count <= 0:
        return []
    per_channel = max(1, token_count * bytes_per_symbol)
    ch_target = max(1, target_bytes // per_channel)
    ch_max = max(1, max_bytes // per_channel)
    ch_min = max(1, min_bytes // per_channel)
    head_bytes = _box_bytes(token_count, head_dim, bytes_per_symbol)

    plan: list[PlannedChunk] = []

    def emit(h0: int, h1: int, c0: int, c1: int, channels: int) -> None:
        plan.append(PlannedChunk(
            chunk_id=len(plan),
            layout=ChunkLayout(
                layer_index=layer_index,
                head_start=h0, head_end=h1,
                channel_start=c0, channel_end=c1,
                token_start=0, token_end=token_count,
                unpacked_bytes=_box_bytes(token_count, channels, bytes_per_symbol),
            ),
        ))

    head = 0
    while head < num_heads:
        heads_left = num_heads - head
        if head_bytes < target_bytes and heads_left > 1:
            group = min(ch_target // head_dim, ch_max // head_dim, heads_left)
            group = min(heads_left, max(1, group))
            while (group < heads_left
                   and _box_bytes(token_count, group * head_dim, bytes_per_symbol) < min_bytes):
                group += 1
            emit(head, head + group, 0, head_dim, group * head_dim)
            head += group
            continue
        step = max(1, min(ch_target, ch_max))
        channel = 0
        while channel < head_dim:
            left = head_dim - channel
            width = min(left, step)
            if left > width:
                width = min(max(width, ch_min), left)
            emit(head, head + 1, channel, channel + width, width)
            channel += width
        head += 1
    return plan

"""Layer-wise restore pipeline: overlapped copy + fused restore (layers dealt
to 2 or 3 lane streams, each lane's slot reused every n layers) gives the
same cache bytes as the direct restore and as the oracle's unpack + scatter
(bitpack_layout_cuda.cu:91-128, benchmark_utils.py:350-444), from pinned
streams and from staging fills."""
import numpy as np
import pytest
import torch

from oracle import oracle
from origami_amd.layout import kv_symbol_layout
from origami_amd.lossless import native_gpu
from origami_amd.lossless.chunking import plan_head_channel_chunks
from origami_amd.restore_pipeline import LayerRestorePipeline

pytestmark = pytest.mark.gpu


def _specs(T2, H, C, target):
    return [[c.layout.head_start, c.layout.head_end, c.layout.channel_start,
             c.layout.channel_end, 0, T2]
            for c in plan_head_channel_chunks(layer_index=0, num_heads=H, head_dim=C,
                                              token_count=T2, bytes_per_symbol=1,
                                              min_bytes=target, target_bytes=target,
                                              max_bytes=target)]


@pytest.mark.parametrize("lanes", [2, 3])
@pytest.mark.parametrize("mode", ["pinned", "filled"])
def test_pipeline_matches_direct_restore(cuda_device, mode, lanes):
    g = torch.Generator().manual_seed(3)
    L, T, H, C, bs = 7, 1000, 4, 256, 16
    nblk = -(-T // bs)
    NB = nblk + 9
    lay = kv_symbol_layout(T, H, C, 8, _specs(2 * T, H, C, 1 << 16))
    streams = [torch.randint(0, 256, (lay.stream_bytes,), dtype=torch.uint8, generator=g)
               for _ in range(L)]
    ids_host = [torch.randperm(NB, generator=g)[:nblk] for _ in range(L)]
    ids = [native_gpu.block_ids_tensor(i, cuda_device) for i in ids_host]
    expect, got, oracle_caches = [], [], []
    for layer in range(L):
        c = torch.zeros((2, NB, bs, H, C), dtype=torch.uint8, device=cuda_device)
        native_gpu.unpack_to_kv_cache(streams[layer].to(cuda_device), lay, T, c, ids[layer])
        expect.append(c)
        got.append(torch.zeros_like(c))
        o = np.zeros((2, NB, bs, H, C), dtype=np.uint8)
        oracle.restore_layer(streams[layer].numpy(), lay.offsets, 8, lay.specs, T, H, C,
                             ids_host[layer].numpy(), o)
        oracle_caches.append(o)
    pipe = LayerRestorePipeline(cuda_device, lay.stream_bytes, num_lanes=lanes)
    events = []
    pinned = [s.pin_memory() for s in streams]
    for layer in range(L):
        if mode == "pinned":
            ev = pipe.restore_pinned(pinned[layer], lay, T, got[layer], ids[layer])
        else:
            ev = pipe.restore_filled(lambda buf, s=streams[layer]: buf.copy_(s), lay, T,
                                     got[layer], ids[layer])
        events.append(ev)
    # consumers wait per layer on the current stream, as wait_for_layer_load does
    for layer in range(L):
        torch.cuda.current_stream(cuda_device).wait_event(events[layer])
        assert torch.equal(got[layer], expect[layer]), layer
        assert np.array_equal(got[layer].cpu().numpy(), oracle_caches[layer]), layer

"""Concurrent restores through the connector: requests of growing length in
one batch run on separate executor threads (batched restores switched off,
origami_batch_restores), so a larger request replaces the
device's restore pipeline while a smaller one may still be submitting to the
old one.  Every restored block must equal the saved source block, blocks
outside the destination tables stay zero, and the per-layer metric rows
(layer_ready, lossless_decompress, h2d_copy, bitunpack_cuda) are written with
event-timed milliseconds."""
import json
import time
import types

import numpy as np
import pytest
import torch

from oracle import oracle
from origami_amd.connector import KVConnectorRole, OrigamiConnector
from origami_amd.metadata import (OrigamiConnectorMetadata, OrigamiRestoreRequest,
                                  OrigamiSaveRequest)

pytestmark = pytest.mark.gpu


def _connector(ns, metrics_dir=""):
    cfg = types.SimpleNamespace(kv_transfer_config=types.SimpleNamespace(
        kv_connector_extra_config={
            "origami_quantizer": "raw_byte_planes", "origami_lossless_cpu_backend": "zlib",
            "origami_store_uri": f"memory://{ns}", "origami_chunk_min_bytes": 1 << 16,
            "origami_chunk_target_bytes": 1 << 16, "origami_chunk_max_bytes": 1 << 16,
            "origami_qat_threads": 8, "origami_metrics_dir": metrics_dir,
            "origami_batch_restores": False}))
    return OrigamiConnector(cfg, KVConnectorRole.WORKER)


def test_concurrent_growing_restores(cuda_device, tmp_path):
    g = torch.Generator(device=cuda_device).manual_seed(21)
    L, NB, bs, H, D = 6, 400, 16, 4, 128
    lengths = [8, 24, 56, 120]  # blocks per request, each larger than the last
    names = [f"model.layers.{i}.self_attn.attn" for i in range(L)]
    src = {n: torch.randn((2, NB, bs, H, D), generator=g, device=cuda_device,
                          dtype=torch.bfloat16) for n in names}
    perm = torch.randperm(NB, generator=g, device=cuda_device).tolist()
    src_ids, at = [], 0
    for n_blk in lengths:
        src_ids.append(perm[at:at + n_blk])
        at += n_blk
    ns = "concurrent-growing"
    saver = _connector(ns)
    saver.register_kv_caches(src)
    saver.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_save={
        f"s{i}": OrigamiSaveRequest(request_id=f"s{i}", cache_key=f"ck{i}",
                                    block_ids_per_group=(tuple(ids),), num_tokens=len(ids) * bs)
        for i, ids in enumerate(src_ids)}))
    saver.start_load_kv(None)
    for n in names:
        saver.save_kv_layer(n, src[n], None)
    saver.wait_for_save()

    # destination tables: disjoint, drawn from another permutation
    perm2 = torch.randperm(NB, generator=g, device=cuda_device).tolist()
    dst_ids, at = [], 0
    for n_blk in lengths:
        dst_ids.append(perm2[at:at + n_blk])
        at += n_blk
    dst = {n: torch.zeros_like(src[n]) for n in names}
    loader = _connector(ns, metrics_dir=str(tmp_path))
    loader.register_kv_caches(dst)
    loader.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_restore={
        f"r{i}": OrigamiRestoreRequest(request_id=f"r{i}", cache_key=f"ck{i}",
                                       block_ids_per_group=(tuple(ids),),
                                       num_tokens=len(ids) * bs)
        for i, ids in enumerate(dst_ids)}))
    loader.start_load_kv(None)
    for n in names:
        loader.wait_for_layer_load(n)
    torch.cuda.synchronize(cuda_device)
    for n in names:
        got = dst[n].view(torch.uint8).cpu().numpy()
        expect = np.zeros_like(got)
        src_np = src[n].view(torch.uint8).cpu().numpy()
        for s_ids, d_ids in zip(src_ids, dst_ids):
            # the oracle's block scatter of the saved blocks' bytes
            tok = oracle.gather_kv_cache(src_np, np.asarray(s_ids))
            oracle.scatter_kv_cache(tok, len(s_ids) * bs, H, 2 * D, np.asarray(d_ids), expect)
        assert np.array_equal(got, expect), n

    finished = set()
    for _ in range(500):
        finished |= loader.get_finished(set())[1]
        if len(finished) == len(lengths):
            break
        time.sleep(0.01)
    assert finished == {f"r{i}" for i in range(len(lengths))}
    worker = loader.connector_worker
    largest = 2 * lengths[-1] * bs * H * 2 * D
    assert worker._pipelines.current()[0].slot_bytes >= largest
    worker.shutdown()
    worker._pipelines.prune()
    assert worker._pipelines.retired() == []

    rows = [json.loads(x) for x in (tmp_path / "origami_metrics.jsonl").read_text().splitlines()]
    kinds = {}
    for r in rows:
        kinds.setdefault(r["type"], []).append(r)
    per_layer = len(names) * len(lengths)
    for kind in ("layer_ready", "lossless_decompress", "h2d_copy", "bitunpack_cuda"):
        assert len(kinds.get(kind, [])) == per_layer, kind
    for r in kinds["bitunpack_cuda"] + kinds["h2d_copy"]:
        assert r["ms"] > 0 and r["gbps"] > 0
        assert r["request_id"] in {f"r{i}" for i in range(len(lengths))}
    assert all(r["timing_complete"] for r in kinds["h2d_copy"])

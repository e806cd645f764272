"""Batched restore through the connector: one start_load_kv with 8 requests
of ragged lengths whose block tables share a prefix (the same destination
blocks in every table, as vLLM's prefix caching shares full blocks).  The
worker restores each layer of the batch with one H2D copy and one batched
launch (the reference restores request by request, worker.py:426-481,
796-897).  The restored caches must equal the oracle's unpack + scatter of
the stored chunk streams, request after request (bitpack_layout_cuda.cu:91-128,
benchmark_utils.py:350-444), byte for byte, and hold the saved source blocks;
blocks outside every table stay untouched."""
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


def _connector(ns, metrics_dir="", batch=True):
    cfg = types.SimpleNamespace(kv_transfer_config=types.SimpleNamespace(
        kv_connector_extra_config={
            "origami_quantizer": "raw_byte_planes", "origami_lossless_cpu_backend": "zlib",
            "origami_store_uri": f"memory://{ns}", "origami_chunk_min_bytes": 1 << 16,
            "origami_chunk_target_bytes": 1 << 16, "origami_chunk_max_bytes": 1 << 16,
            "origami_qat_threads": 8, "origami_metrics_dir": metrics_dir,
            "origami_batch_restores": batch}))
    return OrigamiConnector(cfg, KVConnectorRole.WORKER)


def _tables(rng, nblks, shared, pool, NB):
    perm = rng.permutation(NB)
    cur, out = pool, []
    for n, k in zip(nblks, shared):
        out.append(np.concatenate([perm[:k], perm[cur:cur + n - k]]).astype(np.int64))
        cur += n - k
    return out


@pytest.mark.parametrize("batch", [True, False])
def test_batched_restore_of_ragged_requests_with_shared_prefix(cuda_device, tmp_path, batch):
    dev = cuda_device
    rng = np.random.default_rng(21)
    L, bs, H, D = 3, 16, 4, 128
    C = 2 * D
    nblks = [int(n) for n in rng.integers(20, 61, 8)]
    shared = [n // 2 for n in nblks]
    pool = max(shared)
    NB = pool + sum(n - k for n, k in zip(nblks, shared)) + 17
    names = [f"model.layers.{i}.self_attn.attn" for i in range(L)]
    g = torch.Generator(device=dev).manual_seed(21)
    src = {n: torch.randn((2, NB, bs, H, D), generator=g, device=dev, dtype=torch.bfloat16)
           for n in names}
    src_tables = _tables(rng, nblks, shared, pool, NB)
    dst_tables = _tables(rng, nblks, shared, pool, NB)
    ns = f"batch-{batch}"

    saver = _connector(ns)
    saver.register_kv_caches(src)
    saver.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_save={
        f"s{i}": OrigamiSaveRequest(request_id=f"s{i}", cache_key=f"ck{i}",
                                    block_ids_per_group=(tuple(int(b) for b in t),),
                                    num_tokens=len(t) * bs)
        for i, t in enumerate(src_tables)}))
    saver.start_load_kv(None)
    for n in names:
        saver.save_kv_layer(n, src[n], None)
    saver.wait_for_save()

    dst = {n: torch.full((2, NB, bs, H, D), 3.0, device=dev, dtype=torch.bfloat16)
           for n in names}
    before = {n: dst[n].view(torch.uint8).cpu().numpy().copy() for n in names}
    metrics = tmp_path / f"m{int(batch)}"
    loader = _connector(ns, str(metrics), batch)
    loader.register_kv_caches(dst)
    loader.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_restore={
        f"r{i}": OrigamiRestoreRequest(request_id=f"r{i}", cache_key=f"ck{i}",
                                       block_ids_per_group=(tuple(int(b) for b in t),),
                                       num_tokens=len(t) * bs)
        for i, t in enumerate(dst_tables)}))
    loader.start_load_kv(None)
    worker = loader.connector_worker
    for n in names:
        loader.wait_for_layer_load(n)
        torch.cuda.synchronize(dev)
        got = dst[n].view(torch.uint8).cpu().numpy()
        expect = before[n].copy()
        for i, t in enumerate(dst_tables):
            lp = worker.store.get(f"ck{i}").layer_payloads[n]
            nat = lp.quant_metadata["origami_native_layout"]
            stream = torch.cat(worker.cpu_codec.decompress_many(
                [c.compressed for c in lp.chunks], [c.unpacked_bytes for c in lp.chunks])).numpy()
            T = nat["token_count"] // 2
            offs = oracle.chunk_offsets(np.asarray(nat["chunk_specs"], np.int64),
                                        np.full(len(nat["chunk_specs"]), 8, np.int64))
            oracle.restore_layer(stream, offs, 8, nat["chunk_specs"], T, H, C, t, expect)
        assert np.array_equal(got, expect), n
        s8 = src[n].view(torch.uint8).cpu().numpy()
        for st, dt in zip(src_tables, dst_tables):
            assert np.array_equal(got[:, dt], s8[:, st]), n
        untouched = sorted(set(range(NB)) - set(np.concatenate(dst_tables).tolist()))
        assert np.array_equal(got[:, untouched], before[n][:, untouched])
    finished = set()
    for _ in range(500):
        finished |= loader.get_finished(set())[1]
        if len(finished) == len(dst_tables):
            break
        time.sleep(0.01)
    assert finished == {f"r{i}" for i in range(len(dst_tables))}
    worker.shutdown()
    rows = [json.loads(x) for x in (metrics / "origami_metrics.jsonl").read_text().splitlines()]
    backends = {r.get("backend") for r in rows if r.get("type") == "bitunpack_cuda"}
    if batch:
        assert backends == {"hip_fused_unpack_scatter_batch"}
        skipped = [r["shared_blocks_skipped"] for r in rows if r.get("type") == "bitunpack_cuda"]
        # a request's leading blocks that an earlier request already restores
        lead = sum(min(shared[i], max(shared[:i])) for i in range(1, len(shared)))
        assert skipped and all(k == lead for k in skipped)
    else:
        assert backends == {"hip_fused_unpack_scatter"}


def test_batched_restore_isolates_a_bad_block_table(cuda_device):
    """Three requests in one start_load_kv; the second names a block id
    outside the cache.  Its layer futures carry the error; the other two are
    still restored by one batched launch per layer and match their saved
    blocks."""
    dev = cuda_device
    rng = np.random.default_rng(33)
    L, bs, H, D, NB = 2, 16, 4, 128, 200
    names = [f"model.layers.{i}.self_attn.attn" for i in range(L)]
    g = torch.Generator(device=dev).manual_seed(33)
    src = {n: torch.randn((2, NB, bs, H, D), generator=g, device=dev, dtype=torch.bfloat16)
           for n in names}
    perm = rng.permutation(NB)
    src_tables = [perm[:30], perm[30:50], perm[50:90]]
    saver = _connector("batch-bad")
    saver.register_kv_caches(src)
    saver.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_save={
        f"s{i}": OrigamiSaveRequest(request_id=f"s{i}", cache_key=f"bk{i}",
                                    block_ids_per_group=(tuple(int(b) for b in t),),
                                    num_tokens=len(t) * bs)
        for i, t in enumerate(src_tables)}))
    saver.start_load_kv(None)
    for n in names:
        saver.save_kv_layer(n, src[n], None)
    saver.wait_for_save()

    perm2 = rng.permutation(NB)
    dst_tables = [perm2[:30], perm2[30:50].copy(), perm2[50:90]]
    dst_tables[1][7] = NB + 5  # outside the cache
    dst = {n: torch.zeros_like(src[n]) for n in names}
    loader = _connector("batch-bad")
    loader.register_kv_caches(dst)
    loader.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_restore={
        f"r{i}": OrigamiRestoreRequest(request_id=f"r{i}", cache_key=f"bk{i}",
                                       block_ids_per_group=(tuple(int(b) for b in t),),
                                       num_tokens=len(t) * bs)
        for i, t in enumerate(dst_tables)}))
    loader.start_load_kv(None)
    worker = loader.connector_worker
    futs = {rid: list(f) for rid, f in worker._pending_request_layer_futures.items()}
    for f in futs["r1"]:
        assert f.exception(timeout=60) is not None
    for rid in ("r0", "r2"):
        for f in futs[rid]:
            res = f.result(timeout=60)
            torch.cuda.current_stream(dev).wait_event(res.event)
    torch.cuda.synchronize(dev)
    for n in names:
        for i in (0, 2):
            got = dst[n][:, dst_tables[i]].view(torch.int16)
            assert torch.equal(got, src[n][:, src_tables[i]].view(torch.int16)), (n, i)
    worker.shutdown()

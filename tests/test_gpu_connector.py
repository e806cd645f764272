"""End-to-end through the connector API on the GPU: save_kv_layer /
wait_for_save packs each layer from the paged cache, start_load_kv /
wait_for_layer_load restores it into another cache through another block
table.  Restored blocks must equal the saved ones byte for byte, and the
stored chunk streams must equal the oracle's pack of the same bytes."""
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


def _connector(quantizer, ns):
    cfg = types.SimpleNamespace(kv_transfer_config=types.SimpleNamespace(
        kv_connector_extra_config={
            "origami_quantizer": quantizer, "origami_lossless_cpu_backend": "zlib",
            "origami_store_uri": f"memory://{ns}", "origami_chunk_min_bytes": 1 << 16,
            "origami_chunk_target_bytes": 1 << 16, "origami_chunk_max_bytes": 1 << 16,
            "origami_qat_threads": 4}))
    return OrigamiConnector(cfg, KVConnectorRole.WORKER)


def _gather(cache, ids, blocks_first):
    return cache[ids] if blocks_first else cache[:, ids]


@pytest.mark.parametrize("quantizer", ["raw_byte_planes", "raw_bytes"])
@pytest.mark.parametrize("blocks_first", [False, True])
def test_save_then_restore_through_connector(cuda_device, quantizer, blocks_first):
    g = torch.Generator(device=cuda_device).manual_seed(7)
    L, NB, bs, H, D, nblk = 4, 80, 16, 8, 128, 50
    shape = (NB, 2, bs, H, D) if blocks_first else (2, NB, bs, H, D)
    names = [f"model.layers.{i}.self_attn.attn" for i in range(L)]
    src = {n: torch.randn(shape, generator=g, device=cuda_device, dtype=torch.bfloat16)
           for n in names}
    src_ids = torch.randperm(NB, generator=g, device=cuda_device)[:nblk].tolist()
    saver = _connector(quantizer, f"e2e-{quantizer}-{blocks_first}")
    saver.register_kv_caches(src)
    saver.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_save={
        "s": OrigamiSaveRequest(request_id="s", cache_key="ck",
                                block_ids_per_group=(tuple(src_ids),), num_tokens=nblk * bs)}))
    saver.start_load_kv(None)  # vLLM calls it every step; the worker takes the metadata here
    for n in names:
        saver.save_kv_layer(n, src[n], None)
    saver.wait_for_save()

    payload = saver.store.get("ck")
    assert sorted(payload.layer_payloads) == sorted(names)
    if quantizer == "raw_byte_planes" and not blocks_first:
        # wire format: decompressed chunks == the oracle's pack of the layer bytes
        lp = payload.layer_payloads[names[1]]
        nat = lp.quant_metadata["origami_native_layout"]
        assert nat["version"] == 2 and nat["source_layout"] == ["token", "head", "head_dim"]
        raw = saver.connector_worker.cpu_codec.decompress_many(
            [c.compressed for c in lp.chunks], [c.unpacked_bytes for c in lp.chunks])
        sym = oracle.gather_kv_cache(src[names[1]].view(torch.uint8).cpu().numpy(),
                                     np.asarray(src_ids))
        ref, _ = oracle.pack_canonical(sym, 8, nat["chunk_specs"], nat["source_shape"],
                                       [0, 1, 2, -1])
        assert np.array_equal(torch.cat(raw).numpy(), ref)

    dst = {n: torch.zeros(shape, device=cuda_device, dtype=torch.bfloat16) for n in names}
    dst_ids = torch.randperm(NB, generator=g, device=cuda_device)[:nblk].tolist()
    loader = _connector(quantizer, f"e2e-{quantizer}-{blocks_first}")
    loader.register_kv_caches(dst)
    loader.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_restore={
        "r": OrigamiRestoreRequest(request_id="r", cache_key="ck",
                                   block_ids_per_group=(tuple(dst_ids),), num_tokens=nblk * bs)}))
    loader.start_load_kv(None)
    for n in names:
        loader.wait_for_layer_load(n)
        got = _gather(dst[n], dst_ids, blocks_first)
        want = _gather(src[n], src_ids, blocks_first)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), n
    finished = set()
    for _ in range(500):
        finished |= loader.get_finished(set())[1]
        if finished:
            break
        time.sleep(0.01)
    assert finished == {"r"}
    # blocks outside the destination table were not touched
    others = sorted(set(range(NB)) - set(dst_ids))
    assert int(_gather(dst[names[0]], others, blocks_first).abs().sum()) == 0


def test_copy_kv_to_hbm_matches_oracle_scatter(cuda_device):
    from origami_amd.benchmark_utils import copy_kv_to_hbm

    rng = np.random.default_rng(2)
    NB, bs, H, D, T = 40, 16, 4, 64, 300
    value = torch.randn(2, T, H, D, dtype=torch.bfloat16)
    ids = rng.permutation(NB)[:-(-T // bs)]
    cache = torch.randn(2, NB, bs, H, D, dtype=torch.bfloat16, device=cuda_device)
    expect = cache.view(torch.uint8).cpu().numpy().copy()
    oracle.scatter_kv_cache(value.view(torch.uint8).numpy(), T, H, 2 * D, ids, expect)
    metric, event = copy_kv_to_hbm(kv_cache=cache, block_ids=ids.tolist(),
                                   value=value.pin_memory(), request_id="r", cache_key="k",
                                   system="origami", layer_name="l0", return_event=True)
    event.synchronize()
    assert metric.bytes_copied == value.numel() * 2 and metric.copy_kind == "dram_to_hbm"
    assert np.array_equal(cache.view(torch.uint8).cpu().numpy(), expect)


@pytest.mark.parametrize("quantizer", ["raw_byte_planes", "cachegen"])
def test_save_then_restore_through_file_store(cuda_device, tmp_path, quantizer):
    """The saver writes a bundle_v1 artifact (manifest.json, payload.bin,
    ORIGQZ1 qat_bundle.dz); a separate connector restores from the files
    alone."""
    g = torch.Generator(device=cuda_device).manual_seed(11)
    L, NB, bs, H, D, nblk = 3, 48, 16, 4, 128, 30
    names = [f"model.layers.{i}.self_attn.attn" for i in range(L)]
    src = {n: torch.randn((2, NB, bs, H, D), generator=g, device=cuda_device,
                          dtype=torch.bfloat16) for n in names}
    src_ids = torch.randperm(NB, generator=g, device=cuda_device)[:nblk].tolist()

    def conn():
        cfg = types.SimpleNamespace(kv_transfer_config=types.SimpleNamespace(
            kv_connector_extra_config={
                "origami_quantizer": quantizer, "origami_lossless_cpu_backend": "zlib",
                "origami_store_uri": f"file://{tmp_path}", "origami_chunk_min_bytes": 1 << 16,
                "origami_chunk_target_bytes": 1 << 16, "origami_chunk_max_bytes": 1 << 16,
                "origami_qat_threads": 4}))
        return OrigamiConnector(cfg, KVConnectorRole.WORKER)

    saver = conn()
    saver.register_kv_caches(src)
    saver.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_save={
        "s": OrigamiSaveRequest(request_id="s", cache_key="ck/file",
                                block_ids_per_group=(tuple(src_ids),), num_tokens=nblk * bs)}))
    saver.start_load_kv(None)
    for n in names:
        saver.save_kv_layer(n, src[n], None)
    saver.wait_for_save()
    bundle = tmp_path / "ck_file"
    assert {p.name for p in bundle.iterdir()} == {"manifest.json", "payload.bin",
                                                  "qat_bundle.dz"}
    assert (bundle / "qat_bundle.dz").read_bytes()[:8] == b"ORIGQZ1\0"

    dst = {n: torch.zeros_like(src[n]) for n in names}
    dst_ids = torch.randperm(NB, generator=g, device=cuda_device)[:nblk].tolist()
    loader = conn()
    loader.register_kv_caches(dst)
    loader.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_restore={
        "r": OrigamiRestoreRequest(request_id="r", cache_key="ck/file",
                                   block_ids_per_group=(tuple(dst_ids),), num_tokens=nblk * bs)}))
    loader.start_load_kv(None)
    ref = None
    if quantizer == "cachegen":
        # the same payload, restored from the in-memory copy the saver made
        ref = {n: torch.zeros_like(src[n]) for n in names}
        payload = loader.store.get_from_qat_bundle("ck/file")
    for n in names:
        loader.wait_for_layer_load(n)
        torch.cuda.synchronize(cuda_device)
        if quantizer == "raw_byte_planes":
            assert torch.equal(dst[n][:, dst_ids].view(torch.int16),
                               src[n][:, src_ids].view(torch.int16)), n
        else:
            lp = payload.layer_payloads[n]
            blob = torch.cat(loader.connector_worker.cpu_codec.decompress_many(
                [c.compressed for c in lp.chunks], [c.unpacked_bytes for c in lp.chunks]))
            adapter = loader.connector_worker.quantizer
            adapter.dequantize(blob.to(cuda_device), lp.quant_metadata, dst_cache=ref[n],
                               block_ids=dst_ids).synchronize()
            assert torch.equal(dst[n].view(torch.int16), ref[n].view(torch.int16)), n


def test_restore_waits_for_work_queued_before_start_load_kv(cuda_device):
    """Restores run on the layer pipeline's own streams; start_load_kv orders
    them after the work already queued on the caller's current stream, as the
    reference's restore on that stream is (worker.py:1087-1248).  Here that
    work is a delayed overwrite of the destination cache: the restored bytes
    must be what is left afterwards.  (The block-table uploads from pageable
    memory on the worker thread's stream also wait for that work today; the
    explicit order keeps the result independent of them.)"""
    g = torch.Generator(device=cuda_device).manual_seed(11)
    L, NB, bs, H, D, nblk = 2, 64, 16, 8, 128, 40
    names = [f"model.layers.{i}.self_attn.attn" for i in range(L)]
    src = {n: torch.randn((2, NB, bs, H, D), generator=g, device=cuda_device,
                          dtype=torch.bfloat16) for n in names}
    src_ids = torch.randperm(NB, generator=g, device=cuda_device)[:nblk].tolist()
    saver = _connector("raw_byte_planes", "ordered")
    saver.register_kv_caches(src)
    saver.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_save={
        "s": OrigamiSaveRequest(request_id="s", cache_key="ck",
                                block_ids_per_group=(tuple(src_ids),), num_tokens=nblk * bs)}))
    saver.start_load_kv(None)
    for n in names:
        saver.save_kv_layer(n, src[n], None)
    saver.wait_for_save()

    dst = {n: torch.zeros_like(src[n]) for n in names}
    dst_ids = torch.randperm(NB, generator=g, device=cuda_device)[:nblk].tolist()
    loader = _connector("raw_byte_planes", "ordered")
    loader.register_kv_caches(dst)
    torch.cuda.synchronize()
    # the caller's stream: a bounded spin of about half a second (calibrated
    # with events), then an overwrite of every block
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    torch.cuda._sleep(1 << 22)
    end.record()
    end.synchronize()
    ms_per_cycle = max(start.elapsed_time(end), 1e-3) / (1 << 22)
    torch.cuda._sleep(int(min(500.0 / ms_per_cycle, 1e11)))
    for n in names:
        dst[n].fill_(3.0)
    loader.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_restore={
        "r": OrigamiRestoreRequest(request_id="r", cache_key="ck",
                                   block_ids_per_group=(tuple(dst_ids),), num_tokens=nblk * bs)}))
    loader.start_load_kv(None)
    for n in names:
        loader.wait_for_layer_load(n)
    torch.cuda.synchronize()
    for n in names:
        assert torch.equal(dst[n][:, dst_ids].view(torch.int16),
                           src[n][:, src_ids].view(torch.int16)), n

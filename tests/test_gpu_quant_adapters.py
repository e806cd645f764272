"""CacheGen and KIVI adapters on the GPU: quantize a layer, restore it through
the fused HIP dequantize-to-cache path and compare with

  * the reference's unfused path (CacheGen: the same float32 expression, so
    bit-exact; KIVI: separate multiply and add and a float16 intermediate,
    so within the tolerance stated in the test), and
  * the CPU oracle (oracle/dequant_oracle.c) applied to the same payload,
    bit-exact;

then run both quantizers end to end through the connector (save_kv_layer /
wait_for_save / start_load_kv / wait_for_layer_load)."""
import time
import types

import numpy as np
import pytest
import torch

from oracle import oracle
from origami_amd.connector import KVConnectorRole, OrigamiConnector
from origami_amd.metadata import (OrigamiConnectorMetadata, OrigamiRestoreRequest,
                                  OrigamiSaveRequest)
from origami_amd.quantization import create_quantizer_adapter

pytestmark = pytest.mark.gpu


def _bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _layer(dev, blocks_first, dtype, NB=40, bs=16, H=4, D=64, seed=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    shape = (NB, 2, bs, H, D) if blocks_first else (2, NB, bs, H, D)
    scale = torch.rand((1,) * 3 + (H, D), generator=g, device=dev) * 3 + 0.1
    return (torch.randn(shape, generator=g, device=dev) * scale).to(dtype)


def _select(cache, ids, blocks_first):
    return cache[ids] if blocks_first else cache[:, ids]


def _assign(cache, ids, value, blocks_first):
    if blocks_first:
        cache[ids] = value
    else:
        cache[:, ids] = value


@pytest.mark.parametrize("blocks_first", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layer", ["model.layers.3.attn", "model.layers.25.attn"])
def test_cachegen_fused_restore_equals_unfused_and_oracle(cuda_device, blocks_first, dtype,
                                                          layer):
    dev = cuda_device
    src = _layer(dev, blocks_first, dtype, seed=1)
    ids = torch.randperm(src.shape[0 if blocks_first else 1], device=dev)[:23]
    a = create_quantizer_adapter("cachegen", {})
    q = a.quantize(_select(src, ids, blocks_first), layer_group=layer)
    m = q.metadata
    assert m["format"] == "cachegen_bitpacked_blob"
    assert m["key_stream_bytes"] == -(-m["key_q_numel"] * m["key_bits"] // 8)
    fused = torch.zeros_like(src)
    a.dequantize(q.symbols, m, dst_cache=fused, block_ids=ids.tolist()).synchronize()
    unfused = torch.zeros_like(src)
    _assign(unfused, ids, a._dequantize_dense(q.symbols, m), blocks_first)
    assert np.array_equal(_bits16(fused), _bits16(unfused))
    expect = np.zeros(src.shape, np.uint16)
    blob = q.symbols.cpu().numpy()
    oracle.cachegen_to_kv_cache(
        blob, m["key_stream_offset"], m["key_stream_bytes"], m["value_stream_offset"],
        m["value_stream_bytes"], m["key_bits"], m["value_bits"], m["key_bins"], m["value_bins"],
        blob[m["key_max_offset"]:m["key_max_offset"] + 2 * m["key_max_numel"]].view(np.float16),
        blob[m["value_max_offset"]:m["value_max_offset"] + 2 * m["value_max_numel"]].view(
            np.float16),
        expect, dtype == torch.bfloat16, blocks_first, ids.tolist(), m["token_count"],
        m["num_heads"], m["head_dim"])
    assert np.array_equal(_bits16(fused), expect)


def _kivi_meta(blob, m, name):
    off, n = m[f"{name}_offset"], m[f"{name}_numel"]
    return blob[off:off + 2 * n].view(np.float16)


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("blocks_first", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_kivi_fused_restore_matches_oracle(cuda_device, bits, blocks_first, dtype):
    dev = cuda_device
    src = _layer(dev, blocks_first, dtype, seed=bits)
    ids = torch.randperm(src.shape[0 if blocks_first else 1], device=dev)[:21]
    a = create_quantizer_adapter("kivi", {"bits": bits, "group_size": 32, "sink_tokens": 48})
    q = a.quantize(_select(src, ids, blocks_first))
    m = q.metadata
    fused = torch.zeros_like(src)
    a.dequantize(q.symbols, m, dst_cache=fused, block_ids=ids.tolist()).synchronize()
    blob = q.symbols.cpu().numpy()
    expect = np.zeros(src.shape, np.uint16)
    oracle.kivi_to_kv_cache(
        blob, m["key_stream_offset"], m["key_stream_bytes"], m["value_stream_offset"],
        m["value_stream_bytes"], bits, True, m["group_size"], m["sink_tokens"],
        *[_kivi_meta(blob, m, k) for k in ("key_scale", "key_zero", "value_scale",
                                          "value_zero", "key_sink", "value_sink")],
        expect, dtype == torch.bfloat16, blocks_first, ids.tolist(), m["token_count"],
        m["num_heads"], m["head_dim"])
    assert np.array_equal(_bits16(fused), expect)
    # the reference's unfused path rounds s * scale and + zero separately and
    # goes through float16 before the cache dtype: within one ulp of the
    # cache dtype (2^-7 relative for bfloat16, 2^-10 for float16)
    unfused = torch.zeros_like(src)
    _assign(unfused, ids, a._dequantize_dense(q.symbols, m), blocks_first)
    f, u = fused.float(), unfused.float()
    rel = 2 ** -7 if dtype == torch.bfloat16 else 2 ** -9
    assert torch.all((f - u).abs() <= f.abs() * rel + 2 ** -14)


def _connector(quantizer, ns, extra):
    cfg = types.SimpleNamespace(kv_transfer_config=types.SimpleNamespace(
        kv_connector_extra_config={
            "origami_quantizer": quantizer, "origami_lossless_cpu_backend": "zlib",
            "origami_store_uri": f"memory://{ns}", "origami_chunk_min_bytes": 1 << 16,
            "origami_chunk_target_bytes": 1 << 16, "origami_chunk_max_bytes": 1 << 16,
            "origami_qat_threads": 4, "origami_quantizer_config": extra}))
    return OrigamiConnector(cfg, KVConnectorRole.WORKER)


@pytest.mark.parametrize("quantizer,extra", [("cachegen", {}),
                                             ("kivi", {"bits": 2, "group_size": 32,
                                                       "sink_tokens": 64}),
                                             ("kivi", {"bits": 3, "group_size": 64,
                                                       "sink_tokens": 16})])
def test_quantized_save_restore_through_connector(cuda_device, quantizer, extra):
    dev = cuda_device
    L, NB, bs, nblk = 3, 60, 16, 37
    names = [f"model.layers.{i}.self_attn.attn" for i in range(L)]
    src = {n: _layer(dev, False, torch.bfloat16, NB=NB, seed=10 + i)
           for i, n in enumerate(names)}
    src_ids = torch.randperm(NB, device=dev)[:nblk].tolist()
    ns = f"q-{quantizer}-{extra.get('bits', 0)}"
    saver = _connector(quantizer, ns, extra)
    saver.register_kv_caches(src)
    saver.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_save={
        "s": OrigamiSaveRequest(request_id="s", cache_key="ck",
                                block_ids_per_group=(tuple(src_ids),), num_tokens=nblk * bs)}))
    saver.start_load_kv(None)
    for n in names:
        saver.save_kv_layer(n, src[n], None)
    saver.wait_for_save()
    payload = saver.store.get("ck")

    dst = {n: torch.zeros_like(src[n]) for n in names}
    dst_ids = torch.randperm(NB, device=dev)[:nblk].tolist()
    loader = _connector(quantizer, ns, extra)
    loader.register_kv_caches(dst)
    loader.bind_connector_metadata(OrigamiConnectorMetadata(reqs_to_restore={
        "r": OrigamiRestoreRequest(request_id="r", cache_key="ck",
                                   block_ids_per_group=(tuple(dst_ids),), num_tokens=nblk * bs)}))
    loader.start_load_kv(None)
    adapter = loader.connector_worker.quantizer
    for n in names:
        loader.wait_for_layer_load(n)
        torch.cuda.synchronize(dev)
        lp = payload.layer_payloads[n]
        blob = torch.cat(loader.connector_worker.cpu_codec.decompress_many(
            [c.compressed for c in lp.chunks], [c.unpacked_bytes for c in lp.chunks]))
        # the restore must equal the adapter's fused restore of the stored blob
        want = torch.zeros_like(dst[n])
        adapter.dequantize(blob.to(dev), lp.quant_metadata, dst_cache=want,
                           block_ids=dst_ids).synchronize()
        assert np.array_equal(_bits16(dst[n]), _bits16(want)), n
        # and approximate the saved values
        err = (dst[n][:, dst_ids].float() - src[n][:, src_ids].float()).abs()
        assert float(err.mean()) < float(src[n][:, src_ids].float().abs().mean()) * 0.9
    finished = set()
    for _ in range(500):
        finished |= loader.get_finished(set())[1]
        if finished:
            break
        time.sleep(0.01)
    assert finished == {"r"}
    assert loader.connector_worker._pipelines, "fused restores run through the layer pipeline"

"""Host-side connector logic (no GPU): configuration, store, codec, value
normalisation and failure delivery through the restore futures."""
import types

import pytest
import torch

from origami_amd.benchmark_utils import normalize_kv_value
from origami_amd.config import OrigamiConfig
from origami_amd.connector import KVConnectorRole, OrigamiConnector
from origami_amd.lossless.cpu_qat import CpuLosslessCodec
from origami_amd.metadata import OrigamiConnectorMetadata, OrigamiPayload, OrigamiRestoreRequest
from origami_amd.quantization import create_quantizer_adapter
from origami_amd.store import InMemoryOrigamiStore, create_origami_store


def _vllm_config(extra):
    return types.SimpleNamespace(kv_transfer_config=types.SimpleNamespace(
        kv_connector_extra_config=extra))


def test_config_reads_reference_keys():
    cfg = OrigamiConfig.from_vllm_config(_vllm_config({
        "origami_quantizer": "raw_byte_planes", "origami_chunk_min_bytes": 4096,
        "origami_chunk_target_bytes": 8192, "origami_chunk_max_bytes": 8192,
        "origami_lossless_cpu_backend": "zlib", "origami_bitunpack_device": "AUTO",
        "origami_qat_threads": 4, "origami_unrelated_knob": 1}))
    assert cfg.quantizer == "raw_byte_planes" and cfg.chunk_target_bytes == 8192
    assert cfg.bitunpack_device == "auto" and cfg.qat_threads == 4
    with pytest.raises(ValueError):
        OrigamiConfig.from_extra_config({"origami_chunk_min_bytes": 10,
                                         "origami_chunk_target_bytes": 5})
    with pytest.raises(ValueError):
        OrigamiConfig.from_extra_config({"origami_layout_policy": "zigzag"})


def test_codec_backends():
    data = torch.randint(0, 4, (100000,), dtype=torch.uint8)
    for backend in ("zlib", "raw"):
        codec = CpuLosslessCodec(backend=backend)
        comp = codec.compress_many([data, data[:10]])
        out = codec.decompress_many(comp, [100000, 10])
        assert torch.equal(out[0], data) and torch.equal(out[1], data[:10])
    assert CpuLosslessCodec(backend="zlib").compress(data).numel() < data.numel() // 2
    with pytest.raises(RuntimeError, match="QAT backend is not available"):
        CpuLosslessCodec(backend="qat")
    assert CpuLosslessCodec(backend="qat", allow_zlib_fallback=True).backend == "zlib"
    with pytest.raises(RuntimeError, match="decoded"):
        CpuLosslessCodec(backend="zlib").decompress(CpuLosslessCodec._zlib_compress(data),
                                                    output_bytes=5)


def test_store_round_trip_and_missing_key():
    store = create_origami_store("memory://t1")
    assert isinstance(store, InMemoryOrigamiStore)
    with pytest.raises(KeyError):
        store.get("nope")
    with pytest.raises(ValueError, match="legacy_pt"):
        create_origami_store("file:///tmp/origami-test-x", artifact_format="legacy_pt")


def test_adapters_byte_views():
    kv = torch.randn(2, 3, 4, 2, 8, dtype=torch.bfloat16)
    planes = create_quantizer_adapter("raw_byte_planes")
    q = planes.quantize(kv)
    assert q.metadata["origami_symbol_shape"] == [2 * 12, 2, 16]
    assert torch.equal(q.symbols.view(torch.bfloat16).reshape(2, 12, 2, 8),
                       kv.reshape(2, 12, 2, 8))
    back = planes.dequantize(q.symbols, q.metadata)
    assert torch.equal(back.view(torch.int16), kv.reshape(2, 12, 2, 8).view(torch.int16))
    raw = create_quantizer_adapter("raw_bytes")
    r = raw.quantize(kv)
    assert r.metadata["origami_symbol_shape"] == [1, 1, kv.numel() * 2]
    assert torch.equal(raw.dequantize(r.symbols, r.metadata).view(torch.int16),
                       kv.view(torch.int16))
    with pytest.raises(ValueError):
        create_quantizer_adapter("kvquant")


def test_normalize_kv_value_shapes():
    cache = torch.zeros(2, 10, 4, 2, 8)
    tok = torch.randn(2, 10, 2, 8)
    assert torch.equal(normalize_kv_value(cache, 3, tok), tok)
    assert torch.equal(normalize_kv_value(cache, 2, tok), tok[:, :8])
    assert torch.equal(normalize_kv_value(cache, 3, tok.permute(0, 2, 1, 3)), tok)
    blocks = torch.randn(2, 3, 4, 2, 8)
    assert torch.equal(normalize_kv_value(cache, 3, blocks), blocks.reshape(2, 12, 2, 8))
    assert torch.equal(normalize_kv_value(cache, 3, blocks.permute(1, 0, 2, 3, 4)),
                       blocks.reshape(2, 12, 2, 8))
    with pytest.raises(ValueError):
        normalize_kv_value(cache, 3, torch.randn(3, 10, 2, 8))


def test_unknown_cache_key_fails_through_futures():
    """store.get raises KeyError on the worker thread; the layer futures carry
    it to wait_for_layer_load and get_finished re-raises it."""
    conn = OrigamiConnector(_vllm_config({"origami_quantizer": "raw_byte_planes",
                                          "origami_lossless_cpu_backend": "zlib",
                                          "origami_store_uri": "memory://cpu-fail"}),
                            KVConnectorRole.WORKER)
    conn.register_kv_caches({"layers.0.attn": torch.zeros(2, 4, 4, 1, 8),
                             "layers.1.attn": torch.zeros(2, 4, 4, 1, 8)})
    md = OrigamiConnectorMetadata(reqs_to_restore={"r1": OrigamiRestoreRequest(
        request_id="r1", cache_key="missing", block_ids_per_group=((0, 1),), num_tokens=8)})
    conn.bind_connector_metadata(md)
    conn.start_load_kv(None)
    with pytest.raises(KeyError):
        conn.wait_for_layer_load("layers.0.attn")
    conn.connector_worker._restore_futures[0].exception()  # wait for the request thread
    with pytest.raises(KeyError):
        conn.get_finished(set())
    with pytest.raises(NotImplementedError):
        conn.build_connector_meta(None)


def test_codec_threads_give_the_same_bytes():
    torch.manual_seed(3)
    data = [torch.randint(0, 8, (int(n),), dtype=torch.uint8) for n in (70000, 1, 5000, 0, 123457)]
    one = CpuLosslessCodec(backend="zlib", threads=1)
    many = CpuLosslessCodec(backend="zlib", threads=4)
    a, b = one.compress_many(data), many.compress_many(data)
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    outs = [torch.empty(int(d.numel()), dtype=torch.uint8) for d in data]
    many.decompress_into(b, outs)
    assert all(torch.equal(x, y) for x, y in zip(outs, data))
    with pytest.raises(RuntimeError, match="decoded"):
        many.decompress_into(b[:2], [torch.empty(5, dtype=torch.uint8), outs[1]])


def test_batched_restore_isolates_a_failing_request():
    """Two requests in one start_load_kv are restored by one batch task; the
    one whose cache key is missing fails through its own futures, the other
    (a payload with no layers to restore) completes."""
    conn = OrigamiConnector(_vllm_config({"origami_quantizer": "raw_byte_planes",
                                          "origami_lossless_cpu_backend": "zlib",
                                          "origami_store_uri": "memory://cpu-batch"}),
                            KVConnectorRole.WORKER)
    names = ["layers.0.attn", "layers.1.attn"]
    conn.register_kv_caches({n: torch.zeros(2, 4, 4, 1, 8) for n in names})
    conn.connector_worker.store.put(OrigamiPayload(
        cache_key="empty", request_id="w", quantizer="raw_byte_planes",
        quantizer_config_hash="", token_start=0, token_count=8))
    md = OrigamiConnectorMetadata(reqs_to_restore={
        "bad": OrigamiRestoreRequest(request_id="bad", cache_key="missing",
                                     block_ids_per_group=((0, 1),), num_tokens=8),
        "ok": OrigamiRestoreRequest(request_id="ok", cache_key="empty",
                                    block_ids_per_group=((2, 3),), num_tokens=8)})
    conn.bind_connector_metadata(md)
    conn.start_load_kv(None)
    worker = conn.connector_worker
    done = {worker._restore_future_to_request_id[f]: f for f in worker._restore_futures}
    assert set(done) == {"bad", "ok"}
    assert isinstance(done["bad"].exception(timeout=30), KeyError)
    assert done["ok"].result(timeout=30) == "ok"
    layer_futs = worker._pending_request_layer_futures["ok"]
    assert all(f.result(timeout=30) is None for f in layer_futs)
    with pytest.raises(KeyError):
        conn.wait_for_layer_load(names[0])

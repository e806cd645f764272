"""bundle_v1 / ORIGQZ1 file store (origami_amd/store.py) on the CPU.

Pinned by the format as the reference writes it (store.py:694-867,
qat_deflate.cpp:1804-1862): a hand-assembled ORIGQZ1 header, payload.bin
offsets and sizes checked against the manifest, the request-group order
(ascending unpacked size, layers sorted as strings), the parser's error
messages, and round trips through both payload.bin and the ORIGQZ1 container.
"""
import json
import time
import zlib

import pytest
import torch

from origami_amd.metadata import ChunkLayout, ChunkRecord, LayerPayload, OrigamiPayload
from origami_amd.store import (LocalFileOrigamiStore, create_origami_store, parse_qat_bundle,
                               qat_bundle_header)


def _payload(codec="zlib", layers=("model.layers.10.attn", "model.layers.2.attn"), seed=0):
    g = torch.Generator().manual_seed(seed)
    p = OrigamiPayload(cache_key="req/ck:1", request_id="r1", quantizer="raw_byte_planes",
                       quantizer_config_hash="h", token_start=0, token_count=64,
                       metadata={"note": "x"})
    for li, name in enumerate(layers):
        chunks = []
        for cid, size in enumerate((4096, 4096, 1000)):
            raw = torch.randint(0, 4, (size,), generator=g, dtype=torch.uint8)
            comp = (torch.frombuffer(bytearray(zlib.compress(raw.numpy().tobytes())),
                                     dtype=torch.uint8) if codec == "zlib" else raw.clone())
            lay = ChunkLayout(layer_index=li, head_start=0, head_end=1, channel_start=cid,
                              channel_end=cid + 1, token_start=0, token_end=64,
                              unpacked_bytes=size)
            chunks.append(ChunkRecord(chunk_id=cid, layout=lay, codec=codec, compressed=comp,
                                      compressed_bytes=int(comp.numel()), unpacked_bytes=size))
        p.layer_payloads[name] = LayerPayload(layer_name=name, quantizer="raw_byte_planes",
                                              quant_metadata={"format": "raw_byte_planes",
                                                              "layer": li},
                                              chunks=chunks[::-1])
    return p


def _same(a: OrigamiPayload, b: OrigamiPayload):
    assert (a.cache_key, a.request_id, a.quantizer, a.token_count) == \
        (b.cache_key, b.request_id, b.quantizer, b.token_count)
    assert sorted(a.layer_payloads) == sorted(b.layer_payloads)
    for name, la in a.layer_payloads.items():
        lb = b.layer_payloads[name]
        assert la.quant_metadata == lb.quant_metadata
        ca = sorted(la.chunks, key=lambda c: c.chunk_id)
        for x, y in zip(ca, lb.chunks):
            assert (x.chunk_id, x.layout, x.codec, x.unpacked_bytes) == \
                (y.chunk_id, y.layout, y.codec, y.unpacked_bytes)
            assert torch.equal(x.compressed, y.compressed)


def test_qat_bundle_header_bytes_by_hand():
    hdr = qat_bundle_header(10, [(10, 4), (7, 3)])
    expect = (b"ORIGQZ1\x00" + (10).to_bytes(4, "little") + (2).to_bytes(4, "little")
              + (17).to_bytes(8, "little") + (10).to_bytes(4, "little") + (4).to_bytes(4, "little")
              + (7).to_bytes(4, "little") + (3).to_bytes(4, "little"))
    assert hdr == expect
    chunk_bytes, records, chunks = parse_qat_bundle(hdr + b"abcdXYZ")
    assert chunk_bytes == 10 and records == [(10, 4), (7, 3)]
    assert [bytes(c) for c in chunks] == [b"abcd", b"XYZ"]


@pytest.mark.parametrize("mutate,msg", [
    (lambda b: b[:20], "too small"),
    (lambda b: b"ORIGQZ2\x00" + b[8:], "magic"),
    (lambda b: b[:8] + (0).to_bytes(4, "little") + b[12:], "chunk_bytes must be positive"),
    (lambda b: b[:12] + (0).to_bytes(4, "little") + b[16:], "chunk_count must be positive"),
    (lambda b: b[:12] + (9).to_bytes(4, "little") + b[16:], "record table exceeds"),
    (lambda b: b[:16] + (18).to_bytes(8, "little") + b[24:], "raw size mismatch"),
    (lambda b: b + b"!", "compressed payload size mismatch"),
    (lambda b: b[:28] + (0).to_bytes(4, "little") + b[32:], "compressed chunk length"),
    (lambda b: b[:24] + (11).to_bytes(4, "little") + b[28:], "raw chunk length"),
])
def test_qat_bundle_parser_rejects_corruption(mutate, msg):
    good = qat_bundle_header(10, [(10, 4), (7, 3)]) + b"abcdXYZ"
    with pytest.raises(RuntimeError, match=msg):
        parse_qat_bundle(mutate(good))


def test_bundle_round_trip_and_layout(tmp_path):
    store = create_origami_store(f"file://{tmp_path}")
    assert isinstance(store, LocalFileOrigamiStore)
    p = _payload()
    store.put(p)
    d = tmp_path / "req_ck_1"
    assert {x.name for x in d.iterdir()} == {"manifest.json", "payload.bin", "qat_bundle.dz"}
    assert store.contains("req/ck:1") and not store.contains("other")
    got = store.get("req/ck:1")
    _same(p, got)
    assert got.metadata["artifact_format"] == "bundle_v1"

    manifest = json.loads((d / "manifest.json").read_text())
    data = (d / "payload.bin").read_bytes()
    # layers sorted as strings ("...10..." before "...2...")
    assert [l["layer_name"] for l in manifest["layers"]] == \
        ["model.layers.10.attn", "model.layers.2.attn"]
    # request groups: ascending unpacked size; offsets tile payload.bin
    assert [g["output_bytes"] for g in manifest["request_groups"]] == [1000, 4096]
    cursor = 0
    for g in manifest["request_groups"]:
        assert g["compressed_offset"] == cursor
        cursor += g["compressed_bytes"]
    assert cursor == len(data)
    for layer in manifest["layers"]:
        lp = p.layer_payloads[layer["layer_name"]]
        for row in layer["chunks"]:
            c = [x for x in lp.chunks if x.chunk_id == row["chunk_id"]][0]
            off, n = row["compressed_offset"], row["compressed_bytes"]
            assert data[off:off + n] == c.compressed.numpy().tobytes()
    qb = manifest["qat_bundle"]
    assert qb["format"] == "ORIGQZ1" and qb["chunks"] == 6 and qb["chunk_bytes"] == 4096
    assert [(r["layer_name"], r["chunk_id"]) for r in qb["refs"]] == [
        ("model.layers.10.attn", 0), ("model.layers.10.attn", 1), ("model.layers.10.attn", 2),
        ("model.layers.2.attn", 0), ("model.layers.2.attn", 1), ("model.layers.2.attn", 2)]
    _, records, _ = parse_qat_bundle((d / "qat_bundle.dz").read_bytes())
    assert [r for r, _ in records] == [4096, 4096, 1000, 4096, 4096, 1000]
    _same(p, store.get_from_qat_bundle("req/ck:1"))


def test_raw_codec_writes_no_qat_bundle(tmp_path):
    store = LocalFileOrigamiStore(tmp_path)
    store.put(_payload(codec="zlib"))
    assert store.qat_bundle_path("req/ck:1").exists()
    store.put(_payload(codec="raw"))  # overwrite: the stale container goes away
    assert not store.qat_bundle_path("req/ck:1").exists()
    assert json.loads(store.manifest_path("req/ck:1").read_text())["qat_bundle"] == {}
    _same(_payload(codec="raw"), store.get("req/ck:1"))
    with pytest.raises(KeyError, match="ORIGQZ1"):
        store.get_from_qat_bundle("req/ck:1")


def test_missing_and_foreign_artifacts(tmp_path):
    store = LocalFileOrigamiStore(tmp_path)
    with pytest.raises(KeyError, match="not found"):
        store.get("nope")
    d = tmp_path / "k"
    d.mkdir()
    (d / "manifest.json").write_text(json.dumps({"format": "bundle_v2"}))
    (d / "payload.bin").write_bytes(b"")
    with pytest.raises(ValueError, match="Unsupported Origami artifact format"):
        store.get("k")


def test_prepare_for_restore_paces_reads(tmp_path):
    store = LocalFileOrigamiStore(tmp_path)
    p = _payload()
    store.put(p)
    size = store.payload_path("req/ck:1").stat().st_size
    metrics = tmp_path / "m.jsonl"
    gbps = size * 8 / 0.2 / 1e9  # paced to take about 0.2 s
    t0 = time.perf_counter()
    got = store.prepare_for_restore("req/ck:1", read_bandwidth_gbps=gbps, metrics_path=metrics,
                                    request_id="r", system="origami")
    assert time.perf_counter() - t0 >= 0.15
    _same(p, got)
    row = json.loads(metrics.read_text().splitlines()[-1])
    assert row["type"] == "ssd_read" and row["bytes_read"] == size

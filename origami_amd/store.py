"""Artifact stores (vllm/.../origami/store.py of the reference).

* InMemoryOrigamiStore (store.py:149-173): payloads by cache key in process
  memory (``memory://namespace``, the reference default).
* LocalFileOrigamiStore (store.py:176-923): the ``bundle_v1`` on-disk format,
  one directory per cache key holding
    - ``payload.bin``: every chunk's compressed bytes, grouped by unpacked
      size (ascending) and within a group in layer-name then chunk-id order;
    - ``qat_bundle.dz`` (when every chunk uses a compressing codec): the
      ``ORIGQZ1`` container, a header ``b"ORIGQZ1\\0"``, ``<u32 chunk_bytes,
      u32 chunk_count, u64 raw_bytes>``, ``chunk_count`` records ``<u32
      raw_len, u32 comp_len>``, then the compressed chunks back to back in
      layer-name then chunk-id order (store.py:694-704, qat_deflate.cpp:
      1804-1910);
    - ``manifest.json``: the payload's fields, per layer the quantizer
      metadata and per chunk its layout, codec, offset and sizes in
      payload.bin, the per-size request groups and the ORIGQZ1 references
      (store.py:706-867).
  Layers are ordered by name as strings, as in the reference, so the
  artifacts of the two implementations are interchangeable.

``legacy_pt`` artifacts (a pickled ``torch.save`` of the payload) are neither
written nor read here: loading one would unpickle arbitrary objects.
"""
from __future__ import annotations

import json
import os
import struct
import time
from dataclasses import asdict
from pathlib import Path
from threading import Lock
from typing import Any

import torch

from origami_amd.benchmark_utils import write_jsonl
from origami_amd.metadata import ChunkLayout, ChunkRecord, LayerPayload, OrigamiPayload

QAT_BUNDLE_MAGIC = b"ORIGQZ1\0"
_QAT_HEADER = struct.Struct("<IIQ")
_QAT_RECORD = struct.Struct("<II")
_QAE_MAX_CHUNK = 64 << 20  # compressed chunk limit of the reference's prepared restore


class OrigamiStore:
    """Store interface (store.py:98-146)."""

    def put(self, payload: OrigamiPayload) -> None:
        raise NotImplementedError

    def get(self, cache_key: str) -> OrigamiPayload:
        raise NotImplementedError

    def contains(self, cache_key: str) -> bool:
        raise NotImplementedError

    def prepare_for_restore(self, cache_key: str, **_kwargs) -> OrigamiPayload:
        return self.get(cache_key)

    def preload_for_restore(self, cache_keys, **_kwargs) -> None:
        return None


class InMemoryOrigamiStore(OrigamiStore):
    _MEMORY: dict[str, OrigamiPayload] = {}
    _MEMORY_LOCK = Lock()

    def __init__(self, namespace: str = "origami"):
        self.namespace = namespace

    def _key(self, cache_key: str) -> str:
        return f"{self.namespace}:{cache_key}"

    def put(self, payload: OrigamiPayload) -> None:
        with self._MEMORY_LOCK:
            self._MEMORY[self._key(payload.cache_key)] = payload

    def get(self, cache_key: str) -> OrigamiPayload:
        with self._MEMORY_LOCK:
            try:
                return self._MEMORY[self._key(cache_key)]
            except KeyError as exc:
                raise KeyError(f"Origami payload not found: {cache_key}") from exc

    def contains(self, cache_key: str) -> bool:
        with self._MEMORY_LOCK:
            return self._key(cache_key) in self._MEMORY

    def clear(self) -> None:
        with self._MEMORY_LOCK:
            for key in [k for k in self._MEMORY if k.startswith(self.namespace + ":")]:
                del self._MEMORY[key]


# ---------------------------------------------------------------------------
# ORIGQZ1 container
# ---------------------------------------------------------------------------

def codec_uses_qat_bundle(codec: str) -> bool:
    """store.py:44-46: every codec but raw/identity and nvCOMP's."""
    c = str(codec).lower()
    return c not in {"raw", "identity"} and not c.startswith("nvcomp")


def qat_bundle_header(chunk_bytes: int, records: list[tuple[int, int]]) -> bytes:
    raw_bytes = sum(raw for raw, _ in records)
    parts = [QAT_BUNDLE_MAGIC, _QAT_HEADER.pack(int(chunk_bytes), len(records), raw_bytes)]
    parts += [_QAT_RECORD.pack(int(raw), int(comp)) for raw, comp in records]
    return b"".join(parts)


def parse_qat_bundle(data: bytes | bytearray | memoryview
                     ) -> tuple[int, list[tuple[int, int]], list[memoryview]]:
    """Validates an ORIGQZ1 container and returns (chunk_bytes, records,
    compressed chunks), with the checks and messages of the reference's
    parser (qat_deflate.cpp:1804-1862)."""
    buf = memoryview(data).cast("B")
    if len(buf) < 24:
        raise RuntimeError("ORIGQZ1 bundle is too small")
    if bytes(buf[:8]) != QAT_BUNDLE_MAGIC:
        raise RuntimeError("invalid ORIGQZ1 bundle magic")
    chunk_bytes, count, raw_bytes = _QAT_HEADER.unpack_from(buf, 8)
    if chunk_bytes <= 0:
        raise RuntimeError("ORIGQZ1 chunk_bytes must be positive")
    if count <= 0:
        raise RuntimeError("ORIGQZ1 chunk_count must be positive")
    header = 24 + 8 * count
    if header > len(buf):
        raise RuntimeError("ORIGQZ1 record table exceeds bundle size")
    records = []
    raw_sum = comp_sum = 0
    for i in range(count):
        raw, comp = _QAT_RECORD.unpack_from(buf, 24 + 8 * i)
        if raw <= 0 or raw > chunk_bytes:
            raise RuntimeError("invalid ORIGQZ1 raw chunk length")
        if comp <= 0:
            raise RuntimeError("invalid ORIGQZ1 compressed chunk length")
        if comp >= _QAE_MAX_CHUNK:
            raise RuntimeError(
                "ORIGQZ1 prepared restore only supports compressed chunks below 64 MiB")
        records.append((raw, comp))
        raw_sum += raw
        comp_sum += comp
    if raw_sum != raw_bytes:
        raise RuntimeError("ORIGQZ1 raw size mismatch")
    if header + comp_sum != len(buf):
        raise RuntimeError("ORIGQZ1 compressed payload size mismatch")
    chunks, cursor = [], header
    for _, comp in records:
        chunks.append(buf[cursor:cursor + comp])
        cursor += comp
    return chunk_bytes, records, chunks


# ---------------------------------------------------------------------------
# bundle_v1 file store
# ---------------------------------------------------------------------------

def _safe_key(cache_key: str) -> str:
    return str(cache_key).replace("/", "_").replace(":", "_")


def _u8_bytes(t: torch.Tensor) -> bytes:
    return t.detach().cpu().to(torch.uint8).reshape(-1).contiguous().numpy().tobytes()


def _atomic_write(path: Path, data: bytes) -> None:
    tmp = path.with_name(path.name + ".tmp")
    with tmp.open("wb") as handle:
        handle.write(data)
    os.replace(tmp, path)


def controlled_read(path: Path, *, bandwidth_gbps: float = 0.0, chunk_bytes: int = 4 << 20,
                    metrics_path: str | Path | None = None, request_id: str = "",
                    cache_key: str = "", system: str = "origami") -> bytes:
    """Reads a file, optionally paced to `bandwidth_gbps` gigabits per second
    (the token-bucket read of benchmark_utils.py:133-230), and records an
    ``ssd_read`` metric row."""
    start_ts = time.time()
    start = time.perf_counter()
    parts, done, io_ms = [], 0, 0.0
    with Path(path).open("rb") as handle:
        while True:
            t0 = time.perf_counter()
            part = handle.read(chunk_bytes)
            io_ms += (time.perf_counter() - t0) * 1e3
            if not part:
                break
            parts.append(part)
            done += len(part)
            if bandwidth_gbps > 0:
                due = done * 8.0 / (bandwidth_gbps * 1e9)
                lag = due - (time.perf_counter() - start)
                if lag > 0:
                    time.sleep(lag)
    ms = (time.perf_counter() - start) * 1e3
    write_jsonl(metrics_path, {
        "type": "ssd_read", "request_id": request_id, "cache_key": cache_key, "system": system,
        "path": str(path), "bytes_read": done, "start_ts": start_ts,
        "end_ts": start_ts + ms / 1e3, "ms": ms, "read_io_ms": io_ms,
        "bandwidth_gbps": float(bandwidth_gbps),
        "effective_limited_read_gbps": done * 8.0 / ms / 1e6 if ms > 0 else 0.0,
    })
    return b"".join(parts)


class LocalFileOrigamiStore(OrigamiStore):
    """bundle_v1 artifacts under `root` (store.py:176-923)."""

    def __init__(self, root: str | Path, artifact_format: str = "bundle_v1"):
        if str(artifact_format) not in {"bundle_v1", "auto"}:
            raise ValueError(f"artifact format {artifact_format!r} is not supported: this build "
                             "reads and writes bundle_v1 only (legacy_pt artifacts are pickles)")
        self.root = Path(root)
        self.root.mkdir(parents=True, exist_ok=True)
        self.artifact_format = str(artifact_format)

    def _bundle_dir(self, cache_key: str) -> Path:
        return self.root / _safe_key(cache_key)

    def manifest_path(self, cache_key: str) -> Path:
        return self._bundle_dir(cache_key) / "manifest.json"

    def payload_path(self, cache_key: str) -> Path:
        return self._bundle_dir(cache_key) / "payload.bin"

    def qat_bundle_path(self, cache_key: str) -> Path:
        return self._bundle_dir(cache_key) / "qat_bundle.dz"

    # -- write ---------------------------------------------------------------

    def put(self, payload: OrigamiPayload) -> None:
        """store.py:706-867.  payload.bin and qat_bundle.dz are written first
        and the manifest last, each through a rename, so a reader never sees
        a manifest without its data."""
        bundle_dir = self._bundle_dir(payload.cache_key)
        bundle_dir.mkdir(parents=True, exist_ok=True)
        names = sorted(payload.layer_payloads)
        entries = [(name, chunk) for name in names
                   for chunk in sorted(payload.layer_payloads[name].chunks,
                                       key=lambda c: int(c.chunk_id))]
        by_size: dict[int, list[tuple[str, ChunkRecord]]] = {}
        for name, chunk in entries:
            by_size.setdefault(int(chunk.unpacked_bytes), []).append((name, chunk))
        blobs = {(name, int(c.chunk_id)): _u8_bytes(c.compressed) for name, c in entries}

        make_qat = bool(entries) and all(codec_uses_qat_bundle(c.codec) for _, c in entries)
        records = [(int(c.unpacked_bytes), len(blobs[(name, int(c.chunk_id))]))
                   for name, c in entries]
        chunk_bytes = max((raw for raw, _ in records), default=1)
        qat_refs = []
        if make_qat:
            body = [qat_bundle_header(chunk_bytes, records)]
            for name, c in entries:
                body.append(blobs[(name, int(c.chunk_id))])
                qat_refs.append({"layer_name": name, "chunk_id": int(c.chunk_id),
                                 "output_bytes": int(c.unpacked_bytes)})
            _atomic_write(self.qat_bundle_path(payload.cache_key), b"".join(body))
        elif self.qat_bundle_path(payload.cache_key).exists():
            self.qat_bundle_path(payload.cache_key).unlink()

        rows: dict[str, dict[int, dict[str, Any]]] = {n: {} for n in names}
        groups: dict[str, dict[int, dict[str, Any]]] = {n: {} for n in names}
        request_groups, data, offset = [], [], 0
        for size in sorted(by_size):
            group_offset, lengths, refs = offset, [], []
            for name, c in by_size[size]:
                blob = blobs[(name, int(c.chunk_id))]
                data.append(blob)
                cid = int(c.chunk_id)
                rows[name][cid] = {
                    "chunk_id": cid, "layout": asdict(c.layout), "codec": str(c.codec),
                    "compressed_offset": offset, "compressed_bytes": len(blob),
                    "unpacked_bytes": int(c.unpacked_bytes),
                }
                g = groups[name].setdefault(size, {"output_bytes": size, "chunk_ids": [],
                                                   "lengths": [], "compressed_offset": offset,
                                                   "compressed_bytes": 0})
                g["chunk_ids"].append(cid)
                g["lengths"].append(len(blob))
                g["compressed_bytes"] += len(blob)
                lengths.append(len(blob))
                refs.append({"layer_name": name, "chunk_id": cid})
                offset += len(blob)
            request_groups.append({"output_bytes": size,
                                   "chunk_ids": [r["chunk_id"] for r in refs], "refs": refs,
                                   "lengths": lengths, "compressed_offset": group_offset,
                                   "compressed_bytes": sum(lengths)})
        _atomic_write(self.payload_path(payload.cache_key), b"".join(data))

        layers = []
        for name in names:
            lp = payload.layer_payloads[name]
            layers.append({
                "layer_name": lp.layer_name, "quantizer": lp.quantizer,
                "quant_metadata": lp.quant_metadata,
                "chunks": [rows[name][cid] for cid in sorted(rows[name])],
                "groups": [groups[name][size] for size in sorted(groups[name])],
            })
        manifest = {
            "format": "bundle_v1",
            "cache_key": payload.cache_key,
            "request_id": payload.request_id,
            "quantizer": payload.quantizer,
            "quantizer_config_hash": payload.quantizer_config_hash,
            "token_start": int(payload.token_start),
            "token_count": int(payload.token_count),
            "metadata": dict(payload.metadata),
            "layers": layers,
            "request_groups": request_groups,
            "qat_bundle": ({
                "format": "ORIGQZ1", "path": "qat_bundle.dz", "chunk_bytes": chunk_bytes,
                "chunks": len(records), "compressed_bytes": sum(c for _, c in records),
                "unpacked_bytes": sum(r for r, _ in records), "refs": qat_refs,
            } if make_qat else {}),
        }
        text = json.dumps(manifest, ensure_ascii=False, indent=2, default=str)
        _atomic_write(self.manifest_path(payload.cache_key), text.encode("utf-8"))

    # -- read ----------------------------------------------------------------

    def read_manifest(self, cache_key: str) -> dict[str, Any]:
        path = self.manifest_path(cache_key)
        if not path.exists():
            raise KeyError(f"Origami bundle manifest not found: {cache_key}")
        with path.open("r", encoding="utf-8") as handle:
            manifest = json.load(handle)
        if manifest.get("format") != "bundle_v1":
            raise ValueError(f"Unsupported Origami artifact format: {manifest.get('format')!r}")
        return manifest

    @staticmethod
    def payload_from_manifest(manifest: dict[str, Any], data: bytes | None,
                              chunk_data: dict[tuple[str, int], Any] | None = None
                              ) -> OrigamiPayload:
        """store.py:880-923.  Compressed bytes come from payload.bin at each
        chunk's offset, or from `chunk_data` keyed by (layer, chunk id)."""
        payload = OrigamiPayload(
            cache_key=str(manifest["cache_key"]), request_id=str(manifest.get("request_id", "")),
            quantizer=str(manifest["quantizer"]),
            quantizer_config_hash=str(manifest.get("quantizer_config_hash", "")),
            token_start=int(manifest.get("token_start", 0)),
            token_count=int(manifest.get("token_count", 0)),
            metadata=dict(manifest.get("metadata") or {}))
        payload.metadata["artifact_format"] = "bundle_v1"
        for layer in manifest["layers"]:
            name = str(layer["layer_name"])
            chunks = []
            for row in layer.get("chunks", []):
                cid, n = int(row["chunk_id"]), int(row["compressed_bytes"])
                if chunk_data is not None:
                    blob = bytes(chunk_data[(name, cid)])
                elif data is not None:
                    off = int(row["compressed_offset"])
                    blob = data[off:off + n]
                else:
                    blob = b""
                if (data is not None or chunk_data is not None) and len(blob) != n:
                    raise RuntimeError(f"Origami bundle chunk {name}:{cid} is truncated")
                compressed = (torch.frombuffer(bytearray(blob), dtype=torch.uint8)
                              if blob else torch.empty((0,), dtype=torch.uint8))
                chunks.append(ChunkRecord(
                    chunk_id=cid, layout=ChunkLayout(**row["layout"]),
                    codec=str(row.get("codec", "qat")), compressed=compressed,
                    compressed_bytes=n, unpacked_bytes=int(row["unpacked_bytes"])))
            payload.layer_payloads[name] = LayerPayload(
                layer_name=name, quantizer=str(layer["quantizer"]),
                quant_metadata=dict(layer.get("quant_metadata") or {}),
                chunks=sorted(chunks, key=lambda c: int(c.chunk_id)))
        return payload

    def get(self, cache_key: str) -> OrigamiPayload:
        manifest = self.read_manifest(cache_key)
        return self.payload_from_manifest(manifest, self.payload_path(cache_key).read_bytes())

    def get_from_qat_bundle(self, cache_key: str) -> OrigamiPayload:
        """The payload rebuilt from qat_bundle.dz and the manifest's ORIGQZ1
        references alone (what the reference's QAT ingress reads,
        store.py:280-429), without payload.bin."""
        manifest = self.read_manifest(cache_key)
        info = manifest.get("qat_bundle") or {}
        if not info:
            raise KeyError(f"Origami bundle {cache_key!r} has no ORIGQZ1 container")
        _, records, chunks = parse_qat_bundle(self.qat_bundle_path(cache_key).read_bytes())
        refs = info.get("refs") or []
        if len(refs) != len(records):
            raise RuntimeError("ORIGQZ1 references do not match the container's chunk count")
        chunk_data = {}
        for ref, (raw, _), blob in zip(refs, records, chunks):
            if int(ref["output_bytes"]) != raw:
                raise RuntimeError("ORIGQZ1 raw chunk length does not match the manifest")
            chunk_data[(str(ref["layer_name"]), int(ref["chunk_id"]))] = blob
        return self.payload_from_manifest(manifest, None, chunk_data)

    def contains(self, cache_key: str) -> bool:
        return self.manifest_path(cache_key).exists() and self.payload_path(cache_key).exists()

    def prepare_for_restore(self, cache_key: str, *, read_bandwidth_gbps: float = 0.0,
                            metrics_path: str | Path | None = None, request_id: str = "",
                            system: str = "origami", **_kwargs) -> OrigamiPayload:
        """The zlib / raw restore read of store.py:433-467: payload.bin,
        paced to read_bandwidth_gbps when that is positive."""
        manifest = self.read_manifest(cache_key)
        data = controlled_read(self.payload_path(cache_key), bandwidth_gbps=read_bandwidth_gbps,
                               metrics_path=metrics_path, request_id=request_id,
                               cache_key=cache_key, system=system)
        return self.payload_from_manifest(manifest, data)


def create_origami_store(uri: str, artifact_format: str = "bundle_v1") -> OrigamiStore:
    """store.py:926-937: memory://namespace, file://root or a plain path."""
    if uri.startswith("memory://"):
        return InMemoryOrigamiStore(uri[len("memory://"):] or "origami")
    if uri.startswith("file://"):
        return LocalFileOrigamiStore(uri[len("file://"):], artifact_format=artifact_format)
    return LocalFileOrigamiStore(uri, artifact_format=artifact_format)

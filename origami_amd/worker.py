"""Connector worker: layer-wise restore and save of KV through the HIP layout path.

Mirrors OrigamiConnectorWorker (vllm/.../origami/worker.py).  The public
methods and their semantics are the reference's:

* start_load_kv (worker.py:426-481): one future per (request, layer); the
  request's restore runs on a worker thread.
* wait_for_layer_load (:553-572): waits for the layer's futures, then makes
  the current (attention) stream wait on the layer's completion event.
* save_kv_layer / wait_for_save (:619-663): per (save request, layer) pack and
  compress, then store.put per cache key.
* get_finished (:2441-2496): request ids whose restore completed; failures
  are re-raised.

What changes is the data path.  A layer saved with the raw_byte_planes
adapter is packed on the GPU straight from the paged cache (fused block gather
+ plane-major pack) and restored through LayerRestorePipeline: decompression
into pinned staging, H2D on a copy stream, fused unpack + block-table scatter on
a compute stream, one event per layer.  Payloads in the reference's raw_bytes
format restore through the same pipeline with a block scatter, and CacheGen
bit-packed and KIVI payloads with their fused unpack + dequantize + scatter
kernels.  Other canonical payloads unpack on the GPU, dequantize through their
adapter and go through copy_kv_to_hbm.
"""
from __future__ import annotations

import hashlib
import json
import time
from concurrent.futures import Future, ThreadPoolExecutor
from dataclasses import dataclass
from pathlib import Path
from threading import Lock
from typing import Any

import numpy as np
import torch

from origami_amd.benchmark_utils import copy_kv_to_hbm, nvtx_range, write_jsonl
from origami_amd.config import OrigamiConfig
from origami_amd.layout import STORAGE_LAYOUT, CanonicalLayout, canonical_axis_sizes
from origami_amd.lossless import native_gpu
from origami_amd.lossless.chunking import PlannedChunk, plan_head_channel_chunks
from origami_amd.lossless.cpu_qat import CpuLosslessCodec
from origami_amd.metadata import (
    ChunkLayout,
    ChunkRecord,
    LayerPayload,
    OrigamiConnectorMetadata,
    OrigamiPayload,
    OrigamiRestoreRequest,
    OrigamiSaveRequest,
)
from origami_amd.quantization import QuantizerAdapter, create_quantizer_adapter
from origami_amd.quantization.raw_tensor import RawBytePlanesAdapter
from origami_amd.restore_pipeline import (LayerRestorePipeline, PipelineRegistry,
                                          order_lanes_after)
from origami_amd.store import OrigamiStore

_NATIVE_LAYOUT_KEY = "origami_native_layout"
# quantized payloads whose restore has a fused HIP dequantize-to-cache path
_FUSED_DEQUANT_FORMATS = ("cachegen_bitpacked_blob", "kivi_structured_blob")


def _layer_index(layer_name: str) -> int:
    """Trailing integer of a layer name (worker.py:63-71)."""
    digits = ""
    for ch in reversed(layer_name):
        if ch.isdigit():
            digits = ch + digits
        elif digits:
            break
    return int(digits) if digits else 0


def _config_hash(config: dict[str, Any]) -> str:
    return hashlib.sha256(json.dumps(config, sort_keys=True, default=str).encode()).hexdigest()


@dataclass
class _LayerLoadResult:
    event: torch.cuda.Event | None = None
    # (metric type, restore, layer payload, fields) rows whose fields hold
    # "_cuda_start_event"/"_cuda_end_event"; read out after the layer's wait
    pending_metrics: list | None = None
    wait_on_current_stream: bool = True


def _ms_since(start: float) -> float:
    return (time.perf_counter() - start) * 1000.0


def _restore_metric_id(restore: OrigamiRestoreRequest | None) -> str:
    if restore is None:
        return ""
    return str(restore.metric_request_id or restore.request_id)


def _layout_to_spec(layout: ChunkLayout) -> list[int]:
    return [int(layout.head_start), int(layout.head_end), int(layout.channel_start),
            int(layout.channel_end), int(layout.token_start), int(layout.token_end)]


class OrigamiConnectorWorker:

    def __init__(self, config: OrigamiConfig, store: OrigamiStore,
                 kv_cache_config: Any | None = None, *, fused_attention_enabled: bool = False):
        self.config = config
        self.store = store
        self.kv_cache_config = kv_cache_config
        if fused_attention_enabled and config.fused_attention == "required":
            raise RuntimeError("Origami fused attention is outside this build")
        self.fused_attention_enabled = False
        self.quantizer: QuantizerAdapter = create_quantizer_adapter(
            config.quantizer, config.quantizer_config)
        self.cpu_codec = CpuLosslessCodec(backend=config.lossless_cpu_backend,
                                          allow_zlib_fallback=config.allow_zlib_fallback,
                                          threads=config.qat_threads)
        self.kv_caches: dict[str, torch.Tensor] = {}
        self.layer_to_cache_group: dict[str, int] = {}
        self._executor = ThreadPoolExecutor(max_workers=max(1, config.qat_threads))
        self._pending_layer_futures: dict[str, list[Future]] = {}
        self._pending_request_layer_futures: dict[str, list[Future]] = {}
        self._restore_futures: list[Future] = []
        self._restore_future_to_request_id: dict[Future, str] = {}
        self._save_futures: list[Future] = []
        self._save_payloads: dict[str, OrigamiPayload] = {}
        self._save_lock = Lock()
        self._pipelines = PipelineRegistry(self._make_pipeline)
        # CUDA-timed metric rows whose end event had not completed when their
        # layer was waited on; written once it has (or at shutdown)
        self._deferred_metrics: list = []
        self._metrics_lock = Lock()
        self._metadata: OrigamiConnectorMetadata | None = None
        self.metrics_path = (str(Path(config.metrics_dir) / "origami_metrics.jsonl")
                             if config.metrics_dir else None)
        if config.bitunpack_device in {"gpu", "cuda", "hip"} and not native_gpu.available():
            raise RuntimeError("Origami GPU bitunpack requested but the HIP layout library "
                               "or a ROCm device is unavailable")

    # ------------------------------------------------------------------ setup

    def register_kv_caches(self, kv_caches: dict[str, torch.Tensor]) -> None:
        self.kv_caches = dict(kv_caches)
        mapping: dict[str, int] = {}
        for idx, group in enumerate(getattr(self.kv_cache_config, "kv_cache_groups", None) or []):
            for name in getattr(group, "layer_names", ()):
                mapping[str(name)] = idx
        for name in self.kv_caches:
            mapping.setdefault(name, 0)
        self.layer_to_cache_group = mapping

    def _make_pipeline(self, index: int, slot_bytes: int) -> LayerRestorePipeline:
        return LayerRestorePipeline(torch.device("cuda", index), slot_bytes,
                                    num_lanes=self.config.restore_slots)

    def _lease_pipeline(self, device: torch.device, slot_bytes: int):
        """Context manager holding the device's pipeline (slots of at least
        slot_bytes) for one submit; a replaced pipeline outlives its leases."""
        index = device.index if device.index is not None else torch.cuda.current_device()
        return self._pipelines.lease(index, int(slot_bytes))

    # --------------------------------------------------------------- restore

    def start_load_kv(self, metadata: OrigamiConnectorMetadata) -> None:
        self._metadata = metadata
        if not metadata.reqs_to_restore:
            return
        restores = list(metadata.reqs_to_restore.values())
        # restores run on the pipelines' lane streams: order them after the
        # work already queued on this thread's current stream, as a restore
        # on that stream would be (worker.py:1087-1248)
        for device in {t.device for t in self.kv_caches.values() if t.is_cuda}:
            order_lanes_after(torch.cuda.current_stream(device), self.config.restore_slots)
        write_jsonl(self.metrics_path, {
            "type": "restore_batch_meta", "system": "origami", "restore_count": len(restores),
            "request_ids": [r.request_id for r in restores],
            "cache_keys": [r.cache_key for r in restores], "ts": time.time()})
        per_request: dict[str, dict[str, Future]] = {}
        for restore in restores:
            layer_futures: dict[str, Future] = {}
            for layer_name in self.kv_caches:
                fut: Future = Future()
                layer_futures[layer_name] = fut
                self._pending_layer_futures.setdefault(layer_name, []).append(fut)
            self._pending_request_layer_futures[restore.request_id] = list(layer_futures.values())
            per_request[restore.request_id] = layer_futures
        if self.config.batch_restores and len(restores) > 1:
            # one task restores the whole batch; each request still has its
            # own layer futures and its own completion future
            done: dict[str, Future] = {}
            for restore in restores:
                rf: Future = Future()
                done[restore.request_id] = rf
                self._restore_futures.append(rf)
                self._restore_future_to_request_id[rf] = restore.request_id
            self._executor.submit(self._restore_batch_layer_futures, restores, per_request, done)
            return
        for restore in restores:
            rf = self._executor.submit(self._restore_request_layer_futures, restore,
                                       per_request[restore.request_id])
            self._restore_futures.append(rf)
            self._restore_future_to_request_id[rf] = restore.request_id

    def _restore_request_layer_futures(self, restore: OrigamiRestoreRequest,
                                       layer_futures: dict[str, Future]) -> str:
        try:
            payload = self.store.prepare_for_restore(
                restore.cache_key, read_bandwidth_gbps=self.config.read_bandwidth_gbps,
                metrics_path=self.metrics_path, request_id=restore.request_id,
                system="origami")
            start_perf = time.perf_counter()
            # fused restores prepared once per (plan, cache geometry, block
            # table) for all layers of the request
            prepared: dict = {}
            try:
                self._restore_layers_in_order(restore, payload, layer_futures, start_perf,
                                              prepared)
            finally:
                for prep in prepared.values():
                    prep.close()
            return restore.request_id
        except Exception as exc:
            for fut in layer_futures.values():
                if not fut.done():
                    fut.set_exception(exc)
            raise

    @staticmethod
    def _fail_request(layer_futures: dict[str, Future], done: Future, exc: BaseException) -> None:
        for fut in layer_futures.values():
            if not fut.done():
                fut.set_exception(exc)
        if not done.done():
            done.set_exception(exc)

    def _restore_batch_layer_futures(self, restores: list[OrigamiRestoreRequest],
                                     layer_futures: dict[str, dict[str, Future]],
                                     done: dict[str, Future]) -> None:
        """The requests of one start_load_kv restored together, layer by layer
        in model order.  The reference runs one thread per request, each
        restoring its layers one by one (worker.py:426-481, 796-897); here a
        layer whose payloads are byte-plane streams is one H2D copy and one
        batched launch for all requests (_restore_layer_batched), and any
        other layer goes request by request through _restore_layer.  Each
        (request, layer) future receives its own outcome; a request whose
        payload cannot be prepared fails alone."""
        prepared: dict = {}
        batches: dict = {}
        try:
            payloads: dict[str, OrigamiPayload] = {}
            for restore in restores:
                rid = restore.request_id
                try:
                    payloads[rid] = self.store.prepare_for_restore(
                        restore.cache_key, read_bandwidth_gbps=self.config.read_bandwidth_gbps,
                        metrics_path=self.metrics_path, request_id=rid, system="origami")
                except Exception as exc:  # noqa: BLE001 - delivered through the futures
                    self._fail_request(layer_futures[rid], done[rid], exc)
            live = [r for r in restores if r.request_id in payloads]
            start_perf = time.perf_counter()
            for layer_name in self.kv_caches:
                entries = [(r, layer_futures[r.request_id][layer_name]) for r in live]
                entries = [(r, f) for r, f in entries if not f.done()]
                if not entries:
                    continue
                try:
                    rest = self._restore_layer_batched(entries, payloads, layer_name,
                                                       start_perf, batches)
                except Exception as exc:  # noqa: BLE001 - delivered through the futures
                    for _, fut in entries:
                        if not fut.done():
                            fut.set_exception(exc)
                    continue
                for restore, fut in rest:
                    try:
                        result = self._restore_layer(restore, payloads[restore.request_id],
                                                     layer_name, start_perf, prepared)
                    except Exception as exc:  # noqa: BLE001
                        fut.set_exception(exc)
                    else:
                        fut.set_result(result)
            for restore in live:
                if not done[restore.request_id].done():
                    done[restore.request_id].set_result(restore.request_id)
        except Exception as exc:  # noqa: BLE001
            for restore in restores:
                self._fail_request(layer_futures[restore.request_id], done[restore.request_id],
                                   exc)
        finally:
            for prep in prepared.values():
                prep.close()

    def _restore_layer_batched(self, entries, payloads, layer_name: str, start_perf: float,
                               batches: dict) -> list:
        """One layer of several requests whose payloads are raw_byte_planes
        streams ([2T, H, D*e] token-major v2 layouts): every request's chunks
        are decompressed into one pinned staging buffer (each stream at a
        256-byte aligned offset), copied to the device in one H2D, and
        restored by one KVRestoreBatch launch (full blocks that several
        requests share are read and written once).  Resolves the futures it
        takes; returns the entries it leaves to the per-request path (other
        formats, a CPU cache, metadata the per-request path rejects, fewer
        than two restorable requests)."""
        kv_cache = self.kv_caches.get(layer_name)
        if kv_cache is None or not kv_cache.is_cuda:
            return entries
        group = self.layer_to_cache_group.get(layer_name, 0)
        _, nb, bs, H, head_bytes = native_gpu.cache_geometry(kv_cache)
        items, rest = [], []
        for restore, fut in entries:
            lp = payloads[restore.request_id].layer_payloads.get(layer_name)
            ids = (restore.block_ids_per_group[group]
                   if group < len(restore.block_ids_per_group) else ())
            meta = lp.quant_metadata if lp is not None else {}
            native = meta.get(_NATIVE_LAYOUT_KEY) or {}
            if (lp is None or not ids or str(meta.get("format", lp.quantizer)) != "raw_byte_planes"
                    or int(native.get("version", 0)) != 2):
                rest.append((restore, fut))
                continue
            layout = CanonicalLayout.make(native["source_shape"], native["source_layout"],
                                          int(native["bits"]), native.get("chunk_specs", []))
            tokens = int(meta.get("token_count", layout.token_count // 2))
            needed = -(-tokens // bs)
            sizes_ok = (len(lp.chunks) == layout.num_chunks and all(
                int(rec.unpacked_bytes) == size
                for rec, size in zip(lp.chunks, layout.chunk_sizes())))
            table = tuple(int(b) for b in ids[:needed])
            if (not sizes_ok or layout.token_count != 2 * tokens or len(ids) < needed
                    or tuple(layout.layout) != ("token", "head", "head_dim")
                    or layout.num_heads != H or layout.head_dim != head_bytes
                    or min(table) < 0 or max(table) >= nb):
                rest.append((restore, fut))  # the per-request path reports the error
                continue
            items.append((restore, fut, lp, layout, tokens, table))
        if len(items) < 2:
            return rest + [(it[0], it[1]) for it in items]

        key = (group, tuple(kv_cache.shape), kv_cache.dtype, kv_cache.device,
               tuple((it[4], it[3].shape, it[3].specs.tobytes(), it[3].bits.tobytes(), it[5])
                     for it in items))
        batch = batches.get(key)
        if batch is None:
            batch = native_gpu.KVRestoreBatch(
                [it[3] for it in items], [it[4] for it in items],
                [np.asarray(it[5], dtype=np.int64) for it in items], kv_cache,
                dedup_shared_blocks=True)
            batches[key] = batch
        bases, total = [], 0
        for it in items:
            bases.append(total)
            total += -(-int(it[3].stream_bytes) // 256) * 256
        views = [(b, int(it[3].stream_bytes)) for b, it in zip(bases, items)]
        timed = self.metrics_path is not None
        fill_ms: dict = {}

        def fill(staging: torch.Tensor) -> None:
            t0 = time.perf_counter()
            comp, outs = [], []
            for it, base in zip(items, bases):
                lp, layout = it[2], it[3]
                off = layout.offsets
                for k in range(layout.num_chunks):
                    comp.append(lp.chunks[k].compressed)
                    outs.append(staging[base + int(off[k]):base + int(off[k + 1])])
            self.cpu_codec.decompress_into(comp, outs)
            fill_ms["ms"] = _ms_since(t0)

        def compute(flat: torch.Tensor) -> None:
            batch.restore([flat[b:b + n] for b, n in views], kv_cache)

        with self._lease_pipeline(kv_cache.device, total) as pipe:
            for lane in pipe.lanes:
                batch.record_stream(lane)
            out = pipe.submit(fill, total, compute, timed=timed)
        results = []
        if timed:
            event, timing = out
            first = items[0]
            stream_bytes = sum(n for _, n in views)
            written = self._written_bytes(kv_cache, sum(len(it[5]) for it in items)
                                          - batch.skipped_blocks)
            ids_list = [it[0].request_id for it in items]
            self._write_restore_metric("lossless_decompress", first[0], first[2], {
                "device": "cpu", "backend": self.cpu_codec.backend,
                "chunks": sum(len(it[2].chunks) for it in items),
                "compressed_bytes": sum(int(r.compressed_bytes) for it in items
                                        for r in it[2].chunks),
                "unpacked_bytes": stream_bytes, "ms": float(fill_ms.get("ms", 0.0)),
                "batch_request_ids": ids_list})
            h2d = {"bytes_copied": total, "bytes": total, "start_ts": time.time(),
                   "device": str(kv_cache.device), "source_device": "cpu (pinned staging)",
                   "copy_kind": "dram_to_hbm", "copy_stream": True,
                   "batch_request_ids": ids_list,
                   "_cuda_start_event": timing.h2d_start, "_cuda_end_event": timing.h2d_end}
            row = {"backend": "hip_fused_unpack_scatter_batch", "batch_request_ids": ids_list,
                   "unpacked_bytes": stream_bytes, "input_bytes": stream_bytes,
                   "output_bytes": written, "bytes": stream_bytes + written,
                   "shared_blocks_skipped": int(batch.skipped_blocks),
                   "_cuda_start_event": timing.compute_start,
                   "_cuda_end_event": timing.compute_end}
            pending = [("h2d_copy", first[0], first[2], h2d),
                       ("bitunpack_cuda", first[0], first[2], row)]
            results.append(_LayerLoadResult(event=event, pending_metrics=pending))
            results += [_LayerLoadResult(event=event) for _ in items[1:]]
        else:
            results = [_LayerLoadResult(event=out) for _ in items]
        for it, result in zip(items, results):
            self._write_restore_metric("layer_ready", it[0], it[2], {
                "ms": _ms_since(start_perf), "chunks": len(it[2].chunks),
                "batched_requests": len(items)})
            it[1].set_result(result)
        return rest

    def _restore_layers_in_order(self, restore: OrigamiRestoreRequest, payload: OrigamiPayload,
                                 layer_futures: dict[str, Future], start_perf: float,
                                 prepared: dict) -> None:
        """Issues the request's layers in model order (the kv_caches order);
        each layer's outcome goes to its future."""
        for layer_name, fut in layer_futures.items():
            if fut.done():
                continue
            try:
                result = self._restore_layer(restore, payload, layer_name, start_perf,
                                             prepared)
            except Exception as exc:  # noqa: BLE001 - delivered through the future
                fut.set_exception(exc)
            else:
                fut.set_result(result)

    def _restore_layer(self, restore: OrigamiRestoreRequest, payload: OrigamiPayload,
                       layer_name: str, start_perf: float | None = None,
                       prepared: dict | None = None) -> _LayerLoadResult | None:
        layer_payload = payload.layer_payloads.get(layer_name)
        if layer_payload is None or layer_name not in self.kv_caches:
            return None
        kv_cache = self.kv_caches[layer_name]
        group = self.layer_to_cache_group.get(layer_name, 0)
        if group >= len(restore.block_ids_per_group):
            return None
        block_ids = list(restore.block_ids_per_group[group])
        if not block_ids:
            return None
        meta = layer_payload.quant_metadata
        native = meta.get(_NATIVE_LAYOUT_KEY) or {}
        fmt = str(meta.get("format", layer_payload.quantizer))
        if not native or int(native.get("version", 0)) != 2:
            raise RuntimeError(f"Origami layer {layer_name!r}: unsupported native layout "
                               f"metadata version {native.get('version')!r}")
        layout = CanonicalLayout.make(native["source_shape"], native["source_layout"],
                                      int(native["bits"]), native.get("chunk_specs", []))
        if len(layer_payload.chunks) != layout.num_chunks:
            raise RuntimeError("Origami native layout metadata chunk count does not match "
                               "payload chunks")
        _, nb, bs, H, head_bytes = native_gpu.cache_geometry(kv_cache)
        with nvtx_range("origami:restore_layer"):
            result = None
            if fmt == "raw_byte_planes" and kv_cache.is_cuda:
                result = self._restore_byte_planes(restore, layer_payload, layout, kv_cache,
                                                   block_ids, bs, nb, meta, group, prepared)
            elif fmt == "raw_bytes" and kv_cache.is_cuda and self._raw_bytes_scatterable(
                    meta, kv_cache, layout):
                result = self._restore_raw_bytes(restore, layer_payload, layout, kv_cache,
                                                 block_ids, nb, meta)
            elif fmt in _FUSED_DEQUANT_FORMATS and kv_cache.is_cuda:
                result = self._restore_fused_dequant(restore, layer_payload, layout, kv_cache,
                                                     block_ids, nb, meta)
            if result is None:
                result = self._restore_generic(restore, layer_payload, layout, kv_cache,
                                               block_ids)
        if start_perf is not None:
            # host-side readiness of the layer: everything for it is enqueued
            # (worker.py:1072-1080)
            self._write_restore_metric("layer_ready", restore, layer_payload, {
                "ms": _ms_since(start_perf), "chunks": len(layer_payload.chunks)})
        return result

    def _fill_from_chunks(self, layer_payload: LayerPayload, layout: CanonicalLayout,
                          timing: dict | None = None):
        sizes = layout.chunk_sizes()
        for rec, size in zip(layer_payload.chunks, sizes):
            if int(rec.unpacked_bytes) != size:
                raise RuntimeError("Origami CUDA packed chunk byte size mismatch")

        def fill(staging: torch.Tensor) -> None:
            start = time.perf_counter()
            off = layout.offsets
            outs = [staging[int(off[k]):int(off[k + 1])] for k in range(layout.num_chunks)]
            self.cpu_codec.decompress_into([r.compressed for r in layer_payload.chunks], outs)
            if timing is not None:
                timing["ms"] = _ms_since(start)
        return fill

    def _submit_layer(self, restore, layer_payload, layout, kv_cache, ids_dev, compute,
                      metric_type: str, fields: dict[str, Any]) -> _LayerLoadResult:
        """Decompress into pinned staging, then H2D + `compute` on the device
        pipeline.  With metrics on, writes the layer's lossless_decompress row
        and returns h2d_copy and `metric_type` rows timed by events, to be read
        out after the layer's wait (worker.py:574-617)."""
        timed = self.metrics_path is not None
        fill_timing: dict | None = {} if timed else None
        with self._lease_pipeline(kv_cache.device, layout.stream_bytes) as pipe:
            pipe.record_stream(ids_dev)
            out = pipe.submit(self._fill_from_chunks(layer_payload, layout, fill_timing),
                              layout.stream_bytes, compute, timed=timed)
        if not timed:
            return _LayerLoadResult(event=out)
        event, timing = out
        compressed = sum(int(r.compressed_bytes) for r in layer_payload.chunks)
        unpacked = int(layout.stream_bytes)
        ms = float(fill_timing.get("ms", 0.0))
        self._write_restore_metric("lossless_decompress", restore, layer_payload, {
            "device": "cpu", "backend": self.cpu_codec.backend,
            "chunks": len(layer_payload.chunks), "compressed_bytes": compressed,
            "unpacked_bytes": unpacked, "ms": ms,
            "compressed_gbps": compressed * 8.0 / ms / 1e6 if ms > 0 else 0.0,
            "unpacked_gbps": unpacked * 8.0 / ms / 1e6 if ms > 0 else 0.0})
        h2d = {"bytes_copied": unpacked, "bytes": unpacked, "start_ts": time.time(),
               "device": str(kv_cache.device), "source_device": "cpu (pinned staging)",
               "copy_kind": "dram_to_hbm", "copy_stream": True,
               "_cuda_start_event": timing.h2d_start, "_cuda_end_event": timing.h2d_end}
        row = {"chunks": len(layer_payload.chunks), "unpacked_bytes": unpacked,
               "input_bytes": unpacked, **fields,
               "_cuda_start_event": timing.compute_start, "_cuda_end_event": timing.compute_end}
        pending = [("h2d_copy", restore, layer_payload, h2d),
                   (metric_type, restore, layer_payload, row)]
        return _LayerLoadResult(event=event, pending_metrics=pending)

    @staticmethod
    def _written_bytes(kv_cache: torch.Tensor, nblk: int) -> int:
        """Bytes a restore writes into the cache: K and V of nblk whole blocks
        ([bs, H, D] each in both cache layouts)."""
        bs, H, D = (int(x) for x in kv_cache.shape[2:])
        return 2 * nblk * bs * H * D * kv_cache.element_size()

    def _restore_byte_planes(self, restore, layer_payload, layout, kv_cache, block_ids, bs, nb,
                             meta, group: int = 0, prepared: dict | None = None):
        tokens = int(meta.get("token_count", layout.token_count // 2))
        if layout.token_count != 2 * tokens:
            raise RuntimeError("raw_byte_planes symbol token axis must be 2 * token_count")
        needed = -(-tokens // bs)
        if len(block_ids) < needed:
            raise RuntimeError("tokens exceed destination block capacity")
        # one prepared restore (plan, checks, device block table) serves every
        # layer of the request with the same chunk plan and cache geometry
        key = (group, tokens, tuple(kv_cache.shape), kv_cache.dtype, kv_cache.device,
               layout.shape, layout.layout, layout.specs.tobytes(), layout.bits.tobytes())
        prep = prepared.get(key) if prepared is not None else None
        if prep is None:
            prep = native_gpu.PreparedRestore(layout, tokens, kv_cache, block_ids[:needed])
            if prepared is not None:
                prepared[key] = prep
        ids_dev = prep.block_ids
        written = self._written_bytes(kv_cache, needed)
        return self._submit_layer(
            restore, layer_payload, layout, kv_cache, ids_dev,
            lambda flat: prep.restore(flat, kv_cache),
            "bitunpack_cuda",
            {"backend": "hip_fused_unpack_scatter", "symbols": int(layout.symbol_count),
             "output_bytes": written, "bytes": int(layout.stream_bytes) + written})

    @staticmethod
    def _raw_bytes_scatterable(meta, kv_cache, layout) -> bool:
        shape = [int(d) for d in meta.get("shape", [])]
        dtype = str(meta.get("dtype", ""))
        return (len(shape) == 5 and shape[0] == 2 and tuple(shape[2:]) == tuple(kv_cache.shape[2:])
                and dtype == str(kv_cache.dtype).replace("torch.", "")
                and layout.shape[0] == 1 and layout.shape[1] == 1 and layout.uniform_bits == 8)

    def _restore_raw_bytes(self, restore, layer_payload, layout, kv_cache, block_ids, nb, meta):
        """Reference raw_bytes payload ([1, 1, N] bits 8 = the blocks' bytes in
        [2, nblk, bs, H, D] order): H2D + block scatter."""
        nblk = int(meta["shape"][1])
        if len(block_ids) < nblk:
            raise RuntimeError("tokens exceed destination block capacity")
        tokens = nblk * int(kv_cache.shape[2])
        ids_dev = native_gpu.block_ids_tensor(block_ids[:nblk], kv_cache.device, nb)
        written = self._written_bytes(kv_cache, nblk)
        return self._submit_layer(
            restore, layer_payload, layout, kv_cache, ids_dev,
            lambda flat: native_gpu.scatter_kv_blocks(flat, tokens, kv_cache, ids_dev),
            "restore_materialize",
            {"backend": "hip_block_scatter", "device": str(kv_cache.device),
             "direct_to_kv_cache": True, "output_bytes": written,
             "bytes": int(layout.stream_bytes) + written})

    def _restore_fused_dequant(self, restore, layer_payload, layout, kv_cache, block_ids, nb,
                               meta):
        """CacheGen bit-packed and KIVI payloads restored whole into whole
        blocks: the blob goes to the device on the copy stream and one fused
        unpack + dequantize + paged scatter runs on the compute stream
        (worker.py:1250-1346 with cachegen_adapter.py:656-819 and
        kivi_adapter.py:537-683).  None when the payload does not qualify."""
        can = getattr(self.quantizer, "can_dequantize_to_cache", None)
        tokens = int(meta.get("token_count", 0) or 0)
        if can is None or tokens <= 0 or tokens != int(restore.num_tokens):
            return None
        if not can(meta, kv_cache, block_ids, tokens=tokens):
            return None
        if list(layout.shape[:2]) != [1, 1] or layout.uniform_bits != 8:
            return None  # the blob must travel as plain bytes
        needed = -(-tokens // int(kv_cache.shape[2]))
        ids_dev = native_gpu.block_ids_tensor(block_ids[:needed], kv_cache.device, nb)
        quantizer = self.quantizer
        written = self._written_bytes(kv_cache, needed)
        return self._submit_layer(
            restore, layer_payload, layout, kv_cache, ids_dev,
            lambda flat: quantizer.dequantize_to_cache(flat, meta, kv_cache, ids_dev, tokens),
            "restore_materialize",
            {"quantizer": quantizer.quantizer_id, "device": str(kv_cache.device),
             "direct_to_kv_cache": True, "h2d_elided": False, "output_bytes": written,
             "bytes": int(layout.stream_bytes) + written})

    def _restore_generic(self, restore, layer_payload, layout, kv_cache, block_ids):
        chunks = self.cpu_codec.decompress_many([r.compressed for r in layer_payload.chunks],
                                                layout.chunk_sizes())
        device = kv_cache.device
        symbols = native_gpu.unpack_canonical_storage_chunks(
            chunks, [int(b) for b in layout.bits], layout.shape, layout.layout, layout.specs,
            device=device)
        native = layer_payload.quant_metadata.get(_NATIVE_LAYOUT_KEY) or {}
        count = int(native.get("symbol_count", symbols.numel()))
        kv = self.quantizer.dequantize(symbols.reshape(-1)[:count],
                                       layer_payload.quant_metadata)
        _, event = copy_kv_to_hbm(kv_cache=kv_cache, block_ids=block_ids, value=kv,
                                  request_id=restore.metric_request_id or restore.request_id,
                                  cache_key=restore.cache_key, system="origami",
                                  layer_name=layer_payload.layer_name,
                                  metrics_path=self.metrics_path, synchronize=False,
                                  return_event=True)
        return _LayerLoadResult(event=event)

    def wait_for_layer_load(self, layer_name: str) -> None:
        for fut in self._pending_layer_futures.pop(layer_name, []):
            result = fut.result()
            event = result.event if isinstance(result, _LayerLoadResult) else result
            wait = not isinstance(result, _LayerLoadResult) or result.wait_on_current_stream
            if event is not None and wait and torch.cuda.is_available():
                torch.cuda.current_stream().wait_event(event)
            if isinstance(result, _LayerLoadResult):
                self._flush_pending_cuda_metrics(result.pending_metrics)

    def _flush_pending_cuda_metrics(self, pending_metrics: list | None,
                                    final: bool = False) -> None:
        """Writes event-timed metric rows (worker.py:574-617): ms from the
        start/end events, and Gbit/s from input_bytes, output_bytes and bytes.
        A row whose end event has not completed yet is kept and written by a
        later call (the reference writes it at once, flagged
        cuda_timing_deferred, and loses the time); with `final`, the events
        are waited for."""
        with self._metrics_lock:
            rows = self._deferred_metrics + list(pending_metrics or [])
            self._deferred_metrics = []
        keep = []
        for row in rows:
            metric_type, restore, layer_payload, fields = row
            start_event = fields.get("_cuda_start_event")
            end_event = fields.get("_cuda_end_event")
            if start_event is None or end_event is None:
                self._write_restore_metric(metric_type, restore, layer_payload, fields)
                continue
            if final:
                end_event.synchronize()
            elif not end_event.query():
                keep.append(row)
                continue
            out = {k: v for k, v in fields.items() if not k.startswith("_cuda_")}
            ms = float(start_event.elapsed_time(end_event))
            out["ms"] = ms
            if metric_type == "h2d_copy":
                out["h2d_ms"] = ms
                out["h2d_gbps"] = int(out.get("bytes_copied", 0)) * 8.0 / ms / 1e6 if ms > 0 else 0.0
                out["end_ts"] = time.time()
                out["timing_complete"] = True
            if ms > 0:
                for key, name in (("input_bytes", "input_gbps"), ("output_bytes", "output_gbps"),
                                  ("bytes", "gbps")):
                    if int(out.get(key, 0) or 0):
                        out[name] = int(out[key]) * 8.0 / ms / 1e6
            self._write_restore_metric(metric_type, restore, layer_payload, out)
        if keep:
            with self._metrics_lock:
                self._deferred_metrics = keep + self._deferred_metrics

    def _write_restore_metric(self, metric_type: str, restore, layer_payload: LayerPayload,
                              fields: dict[str, Any]) -> None:
        """One JSONL row (worker.py:1751-1766)."""
        if not self.metrics_path:
            return
        row = {"type": metric_type, "system": "origami",
               "request_id": _restore_metric_id(restore),
               "cache_key": restore.cache_key if restore is not None else "",
               "layer_name": layer_payload.layer_name}
        row.update(fields)
        write_jsonl(self.metrics_path, row)

    # ------------------------------------------------------------------ save

    def save_kv_layer(self, layer_name: str, kv_layer: torch.Tensor, attn_metadata: Any) -> None:
        del attn_metadata
        if self._metadata is None or not self._metadata.reqs_to_save:
            return
        for save in self._metadata.reqs_to_save.values():
            group = self.layer_to_cache_group.get(layer_name, 0)
            if group >= len(save.block_ids_per_group):
                continue
            block_ids = save.block_ids_per_group[group]
            if not block_ids:
                continue
            if isinstance(self.quantizer, RawBytePlanesAdapter) and kv_layer.is_cuda:
                fut = self._save_byte_planes(save, layer_name, kv_layer, tuple(block_ids))
            else:
                fut = self._save_generic(save, layer_name, kv_layer, tuple(block_ids))
            self._save_futures.append(fut)

    def _plan(self, layer_name: str, token_count: int, heads: int, head_bytes: int
              ) -> list[PlannedChunk]:
        return plan_head_channel_chunks(
            layer_index=_layer_index(layer_name), num_heads=heads, head_dim=head_bytes,
            token_count=token_count, bytes_per_symbol=1,
            min_bytes=self.config.chunk_min_bytes, target_bytes=self.config.chunk_target_bytes,
            max_bytes=self.config.chunk_max_bytes)

    def _native_metadata(self, bits, shape, layout_names, specs, symbol_count) -> dict:
        T, H, C, _, _ = canonical_axis_sizes(shape, layout_names)
        return {
            "version": 2, "bits": int(bits), "source_shape": [int(d) for d in shape],
            "source_layout": list(layout_names), "storage_layout": STORAGE_LAYOUT,
            "token_count": T, "num_heads": H, "head_dim": C, "symbol_count": int(symbol_count),
            "layout_policy": self.config.layout_policy, "bitpack": bool(self.config.bitpack),
            "chunk_specs": [list(map(int, s)) for s in specs],
        }

    def _save_byte_planes(self, save: OrigamiSaveRequest, layer_name: str, kv_layer, block_ids):
        """Fused GPU gather + pack from the paged cache, on the current stream
        (so it follows the model's writes of this layer), then D2H into
        pinned memory; compression runs on a worker thread."""
        _, nb, bs, H, head_bytes = native_gpu.cache_geometry(kv_layer)
        tokens = len(block_ids) * bs  # whole saved blocks (worker.py:1881-1897)
        planned = self._plan(layer_name, 2 * tokens, H, head_bytes)
        specs = [_layout_to_spec(p.layout) for p in planned]
        layout = CanonicalLayout.make([2 * tokens, H, head_bytes], ["token", "head", "head_dim"],
                                      8, specs)
        ids_dev = native_gpu.block_ids_tensor(list(block_ids), kv_layer.device, nb)
        flat = native_gpu.pack_from_kv_cache(kv_layer, ids_dev, tokens, layout)
        host = torch.empty(layout.stream_bytes, dtype=torch.uint8, pin_memory=True)
        host.copy_(flat, non_blocking=True)
        done = torch.cuda.Event()
        done.record()
        meta = RawBytePlanesAdapter.metadata_for(kv_layer.dtype, tokens, H,
                                                 int(kv_layer.shape[4]))
        meta[_NATIVE_LAYOUT_KEY] = self._native_metadata(8, layout.shape, list(layout.layout),
                                                         specs, layout.symbol_count)

        def finish():
            done.synchronize()  # pack and D2H (current stream) have completed
            off = layout.offsets
            raw = [host[int(off[k]):int(off[k + 1])] for k in range(layout.num_chunks)]
            return save, self._layer_payload(save, layer_name, planned, raw, meta)
        return self._executor.submit(finish)

    def _save_generic(self, save: OrigamiSaveRequest, layer_name: str, kv_layer, block_ids):
        """Adapter path: gather the blocks, quantize, pack on the GPU, compress."""
        if kv_layer.is_cuda:
            _, nb, _, _, _ = native_gpu.cache_geometry(kv_layer)
            ids_dev = native_gpu.block_ids_tensor(list(block_ids), kv_layer.device, nb)
            dim = 1 if kv_layer.shape[0] in (1, 2) else 0  # _block_dim (worker.py:1881-1885)
            kv_blocks = torch.index_select(kv_layer, dim, ids_dev)
        else:
            dim = 1 if kv_layer.shape[0] in (1, 2) else 0
            kv_blocks = torch.index_select(kv_layer, dim, torch.tensor(list(block_ids)))
        quantized = self.quantizer.quantize(kv_blocks, layer_group=layer_name)
        flat = quantized.symbols.reshape(-1).to(torch.uint8)
        md = quantized.metadata
        bits = int(md.get("origami_bits", 8)) if self.config.bitpack else 8
        T, H, C, shape, names = canonical_axis_sizes(md["origami_symbol_shape"],
                                                     md["origami_symbol_layout"])
        planned = self._plan(layer_name, T, H, C)
        specs = [_layout_to_spec(p.layout) for p in planned]
        layout = CanonicalLayout.make(shape, names, bits, specs)
        device = kv_layer.device if kv_layer.is_cuda else torch.device("cuda")
        stream, _ = native_gpu.pack_canonical_storage_flat(flat.to(device), bits, shape, names,
                                                           specs)
        host = stream.cpu()
        meta = dict(md)
        meta[_NATIVE_LAYOUT_KEY] = self._native_metadata(bits, shape, names, specs, flat.numel())
        off = layout.offsets
        raw = [host[int(off[k]):int(off[k + 1])] for k in range(layout.num_chunks)]
        return self._executor.submit(lambda: (save, self._layer_payload(save, layer_name,
                                                                        planned, raw, meta)))

    def _layer_payload(self, save, layer_name, planned, raw, meta) -> LayerPayload:
        compressed = self.cpu_codec.compress_many(raw)
        chunks = []
        for idx, (p, r, c) in enumerate(zip(planned, raw, compressed)):
            lay = ChunkLayout(
                layer_index=p.layout.layer_index, head_start=p.layout.head_start,
                head_end=p.layout.head_end, channel_start=p.layout.channel_start,
                channel_end=p.layout.channel_end, token_start=save.token_start,
                token_end=save.token_start + save.num_tokens, unpacked_bytes=int(r.numel()))
            chunks.append(ChunkRecord(chunk_id=idx, layout=lay, codec=self.cpu_codec.backend,
                                      compressed=c, compressed_bytes=int(c.numel()),
                                      unpacked_bytes=int(r.numel())))
        return LayerPayload(layer_name=layer_name, quantizer=self.quantizer.quantizer_id,
                            quant_metadata=meta, chunks=chunks)

    def wait_for_save(self) -> None:
        for fut in self._save_futures:
            save, layer_payload = fut.result()
            with self._save_lock:
                payload = self._save_payloads.get(save.cache_key)
                if payload is None:
                    payload = OrigamiPayload(
                        cache_key=save.cache_key, request_id=save.request_id,
                        quantizer=self.quantizer.quantizer_id,
                        quantizer_config_hash=_config_hash(self.config.quantizer_config),
                        token_start=save.token_start, token_count=save.num_tokens)
                    self._save_payloads[save.cache_key] = payload
                payload.layer_payloads[layer_payload.layer_name] = layer_payload
        for payload in self._save_payloads.values():
            self.store.put(payload)
        self._save_futures.clear()
        self._save_payloads.clear()

    # -------------------------------------------------------------- finished

    def get_finished(self) -> tuple[set[str], set[str]]:
        self._flush_pending_cuda_metrics(None)
        self._pipelines.prune()
        finished_recving: set[str] = set()
        for rf in list(self._restore_futures):
            if not rf.done():
                continue
            req_id = self._restore_future_to_request_id.pop(rf, "")
            self._restore_futures.remove(rf)
            if not req_id:
                continue
            try:
                rf.result()
            except Exception:
                self._pending_request_layer_futures.pop(req_id, None)
                for name, futs in self._pending_layer_futures.items():
                    self._pending_layer_futures[name] = [f for f in futs if not f.done()]
                raise
            layer_futs = self._pending_request_layer_futures.get(req_id, [])
            if layer_futs and all(f.done() for f in layer_futs):
                try:
                    for f in layer_futs:
                        f.result()
                finally:
                    self._pending_request_layer_futures.pop(req_id, None)
                finished_recving.add(req_id)
        return set(), finished_recving

    def flush_metrics(self) -> None:
        """Writes every pending event-timed metric row, waiting for its
        events (rows are otherwise written once their layer's work is
        observed complete)."""
        self._flush_pending_cuda_metrics(None, final=True)

    def shutdown(self) -> None:
        self._executor.shutdown(wait=True)
        for pipe in self._pipelines.pipelines():
            pipe.synchronize()
        self._flush_pending_cuda_metrics(None, final=True)

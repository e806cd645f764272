"""Layer-wise restore pipeline on HIP streams and events.

Replaces the reference's same-stream restore (worker.py:1087-1248 issues the
H2D copies and the unpack/scatter on the worker thread's current stream, so
the copy of layer L+1 waits behind the unpack of layer L) with:

  host stream bytes (pinned)  --H2D, copy stream-->  device slot
      --fused unpack+scatter, compute stream-->  paged KV cache  --> event

* Device slots form a ring; a slot is refilled only after the unpack that
  read it has finished (compute-done event, waited on by the copy stream).
  The slot tensors are marked as used on both side streams (record_stream),
  so when a pipeline is dropped the caching allocator does not hand their
  memory out again before the copies and unpacks queued on them have run.
* Host data already in pinned memory is copied directly (the QAT path of the
  reference decompresses into pinned staging, native_cpu.py:307-316).  Other
  host data is written into a pinned staging buffer taken from a pool; the
  fill (CPU decompression) runs outside the pipeline lock, so concurrent
  requests decompress in parallel.  A staging buffer is refilled only after
  its previous H2D copy has completed.
* Only the enqueue (H2D + unpack + events) is serialised, under a short lock.
* Every layer gets its own completion event; wait_for_layer_load makes the
  attention stream wait on it (worker.py:553-572), so a layer's attention only
  depends on that layer.  With timing on, start/end events around the H2D and
  the unpack are returned too, for deferred readout (worker.py:574-617).

PipelineRegistry holds one pipeline per device for the connector worker.  A
request that needs a larger slot replaces the device's pipeline; the old one
stays referenced until no caller holds a lease on it and its last queued
work has completed.

Pipelines on one device share one copy and one compute stream (created once
per process); all streams are created at the default priority.
"""
from __future__ import annotations

import threading
from collections import deque
from dataclasses import dataclass
from typing import Any, Callable

import torch

from origami_amd import _native
from origami_amd.layout import CanonicalLayout
from origami_amd.lossless import native_gpu


@dataclass
class _Slot:
    device: torch.Tensor
    copy_done: torch.cuda.Event
    compute_done: torch.cuda.Event
    copy_recorded: bool = False
    compute_recorded: bool = False


@dataclass
class LayerTiming:
    """Start/end events of one layer's H2D copy and restore kernel(s)."""
    h2d_start: torch.cuda.Event
    h2d_end: torch.cuda.Event
    compute_start: torch.cuda.Event
    compute_end: torch.cuda.Event


@dataclass
class _Staging:
    host: torch.Tensor
    copied: torch.cuda.Event | None = None  # H2D that last read this buffer


class _StagingPool:
    """Pinned host buffers handed out one per fill; blocks when all are out."""

    def __init__(self, count: int, nbytes: int):
        self._free: deque[_Staging] = deque(
            _Staging(torch.empty(nbytes, dtype=torch.uint8, pin_memory=True))
            for _ in range(count))
        self._cond = threading.Condition()

    def take(self) -> _Staging:
        with self._cond:
            while not self._free:
                self._cond.wait()
            return self._free.popleft()

    def give(self, buf: _Staging) -> None:
        with self._cond:
            self._free.append(buf)
            self._cond.notify()


_stream_lock = threading.Lock()
_side_streams: dict[int, tuple[torch.cuda.Stream, torch.cuda.Stream]] = {}


def side_streams(device: torch.device) -> tuple[torch.cuda.Stream, torch.cuda.Stream]:
    """The (copy, compute) stream pair of `device`, created once per process.
    Every pipeline on the device uses the same pair: streams share the
    process's few hardware queues, and a new pair per pipeline could land
    copy and compute on one queue, which serialises them (measured: one of
    six pipelines created in a row lost the overlap entirely)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    with _stream_lock:
        pair = _side_streams.get(index)
        if pair is None:
            dev = torch.device("cuda", index)
            pair = (torch.cuda.Stream(dev), torch.cuda.Stream(dev))
            _side_streams[index] = pair
        return pair


class LayerRestorePipeline:
    """Copy/compute-overlapped restore of one layer at a time into a cache."""

    def __init__(self, device: torch.device | str, slot_bytes: int, num_slots: int = 3,
                 host_staging: bool = True, grid_limit: int = 0,
                 staging_slots: int | None = None):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("LayerRestorePipeline needs a ROCm device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.slot_bytes = int(slot_bytes)
        self.copy_stream, self.compute_stream = side_streams(self.device)
        self._slots: list[_Slot] = []
        for _ in range(max(2, int(num_slots))):
            dev = torch.empty(self.slot_bytes, dtype=torch.uint8, device=self.device)
            # the slot is written on the copy stream and read on the compute
            # stream: its memory must outlive the work queued there
            dev.record_stream(self.copy_stream)
            dev.record_stream(self.compute_stream)
            self._slots.append(_Slot(dev, torch.cuda.Event(), torch.cuda.Event()))
        n_staging = len(self._slots) if staging_slots is None else max(1, int(staging_slots))
        self._staging = _StagingPool(n_staging, self.slot_bytes) if host_staging else None
        self._next = 0
        self._lock = threading.Lock()
        self._last_done: torch.cuda.Event | None = None
        # Workgroup cap for the restore kernels: a restore hidden behind the
        # next layer's copy needs no more than a share of the GPU, and a
        # thinner launch leaves HBM bandwidth to the concurrent DMA.
        self.grid_limit = int(grid_limit)

    # -- internals (called with self._lock held) -----------------------------

    def _h2d(self, slot: _Slot, src: torch.Tensor, nbytes: int,
             timing: LayerTiming | None) -> torch.Tensor:
        dst = slot.device[:nbytes]
        with torch.cuda.stream(self.copy_stream):
            if slot.compute_recorded:
                self.copy_stream.wait_event(slot.compute_done)  # device slot free
            if timing is not None:
                timing.h2d_start.record(self.copy_stream)
            dst.copy_(src[:nbytes], non_blocking=True)
            slot.copy_done.record(self.copy_stream)
            slot.copy_recorded = True
            if timing is not None:
                timing.h2d_end.record(self.copy_stream)
        return dst

    def _compute(self, slot: _Slot, flat: torch.Tensor,
                 compute: Callable[[torch.Tensor], None],
                 timing: LayerTiming | None) -> torch.cuda.Event:
        done = torch.cuda.Event()
        with torch.cuda.stream(self.compute_stream):
            self.compute_stream.wait_event(slot.copy_done)
            if timing is not None:
                timing.compute_start.record(self.compute_stream)
            previous = _native.set_rows_grid_limit(self.grid_limit)
            try:
                compute(flat)
            finally:
                _native.set_rows_grid_limit(previous)
            slot.compute_done.record(self.compute_stream)
            slot.compute_recorded = True
            if timing is not None:
                timing.compute_end.record(self.compute_stream)
            done.record(self.compute_stream)
        self._last_done = done
        return done

    def _enqueue(self, src: torch.Tensor, nbytes: int, compute: Callable[[torch.Tensor], None],
                 timing: LayerTiming | None) -> tuple[torch.cuda.Event, torch.cuda.Event]:
        with self._lock:
            slot = self._slots[self._next % len(self._slots)]
            self._next += 1
            flat = self._h2d(slot, src, nbytes, timing)
            copied = torch.cuda.Event()
            copied.record(self.copy_stream)
            return self._compute(slot, flat, compute, timing), copied

    # -- public API ----------------------------------------------------------

    def submit(self, source: torch.Tensor | Callable[[torch.Tensor], None], nbytes: int,
               compute: Callable[[torch.Tensor], None], *, timed: bool = False
               ) -> torch.cuda.Event | tuple[torch.cuda.Event, LayerTiming]:
        """One layer: bring `nbytes` of stream to the device and run `compute`
        on the device copy (on the compute stream).  `source` is either a
        pinned host tensor (copied directly; the caller keeps it alive until
        the returned event completes) or a callable that writes the stream into
        a pinned staging buffer.  The fill runs without any pipeline lock;
        the enqueue of one layer is never interleaved with another's.  With
        `timed`, returns (event, LayerTiming)."""
        nbytes = int(nbytes)
        if nbytes > self.slot_bytes:
            raise RuntimeError("layer stream larger than the pipeline slot")
        timing = None
        if timed:
            timing = LayerTiming(*(torch.cuda.Event(enable_timing=True) for _ in range(4)))
        if callable(source):
            if self._staging is None:
                raise RuntimeError("pipeline was built without host staging")
            buf = self._staging.take()
            try:
                if buf.copied is not None:
                    buf.copied.synchronize()  # its previous H2D has read it
                staging = buf.host[:nbytes]
                source(staging)
                done, buf.copied = self._enqueue(staging, nbytes, compute, timing)
            finally:
                self._staging.give(buf)
        else:
            if source.numel() < nbytes:
                raise RuntimeError("host stream shorter than the layer stream")
            done, _ = self._enqueue(source.reshape(-1), nbytes, compute, timing)
        return (done, timing) if timed else done

    def restore_pinned(self, host_stream: torch.Tensor, layout: CanonicalLayout, tokens: int,
                       kv_cache: torch.Tensor, block_ids: torch.Tensor) -> torch.cuda.Event:
        """Restores one layer from a pinned host stream (fused unpack+scatter)."""
        return self.submit(host_stream, layout.stream_bytes,
                           lambda flat: native_gpu.unpack_to_kv_cache(flat, layout, tokens,
                                                                      kv_cache, block_ids))

    def restore_filled(self, fill: Callable[[torch.Tensor], None], layout: CanonicalLayout,
                       tokens: int, kv_cache: torch.Tensor,
                       block_ids: torch.Tensor) -> torch.cuda.Event:
        """Restores one layer whose stream `fill` writes into pinned staging
        (e.g. CPU decompression straight into pinned memory)."""
        return self.submit(fill, layout.stream_bytes,
                           lambda flat: native_gpu.unpack_to_kv_cache(flat, layout, tokens,
                                                                      kv_cache, block_ids))

    def copy_only(self, host_stream: torch.Tensor, nbytes: int) -> torch.cuda.Event:
        """H2D of one stream into a slot with no compute (the copy-only
        baseline the pipeline is measured against)."""
        with self._lock:
            slot = self._slots[self._next % len(self._slots)]
            self._next += 1
            self._h2d(slot, host_stream.reshape(-1), nbytes, None)
            done = torch.cuda.Event()
            done.record(self.copy_stream)
            self._last_done = done
            return done

    def idle(self) -> bool:
        """True when every layer submitted so far has completed on the GPU."""
        with self._lock:
            last = self._last_done
        return last is None or last.query()

    def synchronize(self) -> None:
        self.copy_stream.synchronize()
        self.compute_stream.synchronize()


class PipelineRegistry:
    """One restore pipeline per device, grown on demand.

    `lease(index, slot_bytes)` returns a context manager yielding a pipeline
    whose slots hold at least `slot_bytes`.  A larger request replaces the
    device's pipeline; the replaced one is retired, not dropped: it stays
    referenced while any caller still holds a lease on it or work it queued is
    still pending (`idle()` is False), and is released on a later lease or
    prune once neither holds.  `factory(index, slot_bytes)` builds pipelines;
    it is injectable so the bookkeeping is testable without a GPU."""

    def __init__(self, factory: Callable[[int, int], Any]):
        self._factory = factory
        self._lock = threading.Lock()
        self._current: dict[int, Any] = {}
        self._leases: dict[int, int] = {}  # id(pipeline) -> active leases
        self._retired: list[Any] = []

    def _prune_locked(self) -> None:
        keep = []
        for pipe in self._retired:
            if self._leases.get(id(pipe), 0) > 0 or not pipe.idle():
                keep.append(pipe)
            else:
                self._leases.pop(id(pipe), None)
        self._retired = keep

    def acquire(self, index: int, slot_bytes: int) -> Any:
        with self._lock:
            self._prune_locked()
            pipe = self._current.get(index)
            if pipe is None or pipe.slot_bytes < slot_bytes:
                if pipe is not None:
                    self._retired.append(pipe)
                pipe = self._factory(index, slot_bytes)
                self._current[index] = pipe
            self._leases[id(pipe)] = self._leases.get(id(pipe), 0) + 1
            return pipe

    def release(self, pipe: Any) -> None:
        with self._lock:
            n = self._leases.get(id(pipe), 0) - 1
            if n < 0:
                raise RuntimeError("pipeline released more often than leased")
            self._leases[id(pipe)] = n
            self._prune_locked()

    def lease(self, index: int, slot_bytes: int):
        registry = self

        class _Lease:
            def __enter__(self_inner):
                self_inner.pipe = registry.acquire(index, slot_bytes)
                return self_inner.pipe

            def __exit__(self_inner, *exc):
                registry.release(self_inner.pipe)
                return False

        return _Lease()

    def prune(self) -> None:
        with self._lock:
            self._prune_locked()

    def current(self) -> dict[int, Any]:
        with self._lock:
            return dict(self._current)

    def retired(self) -> list[Any]:
        with self._lock:
            return list(self._retired)

    def pipelines(self) -> list[Any]:
        with self._lock:
            return list(self._current.values()) + list(self._retired)

    def __bool__(self) -> bool:
        with self._lock:
            return bool(self._current)

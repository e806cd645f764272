"""Layer-wise restore pipeline on HIP streams and events.

Replaces the reference's same-stream restore (worker.py:1087-1248 issues the
H2D copies and the unpack/scatter on the worker thread's current stream, so
the copy of layer L+1 waits behind the unpack of layer L) with lanes:

  host stream bytes (pinned)  --H2D-->  lane slot  --fused unpack+scatter-->
      paged KV cache  --> event          (all on the lane's stream)

* A lane is a stream with its own device slot.  Layer i goes to lane
  i mod n: its H2D copy, then its restore, then its completion event, all on
  that one stream.  The copy of layer i+1 runs on the next lane while layer
  i's restore runs, so with n >= 2 lanes the restores hide behind the copies;
  a lane's slot is refilled only after the restore that read it, by stream
  order alone.  No event crosses streams: a restore stream that waits on a
  copy stream's event made each 512 MiB copy about 60 us longer (80 layers of
  the Llama-3-70B geometry: 755.9 ms against 750.9 ms for the bare copies),
  while 2 lanes took 750.4 ms with every restore included.
* The slot tensors are marked as used on their lane (record_stream), so when
  a pipeline is dropped the caching allocator does not hand their memory out
  again before the work queued there has run.
* Host data already in pinned memory is copied directly (the QAT path of the
  reference decompresses into pinned staging, native_cpu.py:307-316).  Other
  host data is written into a pinned staging buffer taken from a pool; the
  fill (CPU decompression) runs outside the pipeline lock, so concurrent
  requests decompress in parallel.  A staging buffer is refilled only after
  its previous H2D copy has completed.
* Only the enqueue (H2D + restore + events) is serialised, under a short lock.
* Every layer gets its own completion event; wait_for_layer_load makes the
  attention stream wait on it (worker.py:553-572), so a layer's attention only
  depends on that layer.  With timing on, start/end events around the H2D and
  the restore are returned too, for deferred readout (worker.py:574-617).

PipelineRegistry holds one pipeline per device for the connector worker.  A
request that needs a larger slot replaces the device's pipeline; the old one
stays referenced until no caller holds a lease on it and its last queued
work has completed.

Pipelines on one device share the device's lane streams (created once per
process); all streams are created at the default priority.
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
_lanes: dict[int, list[torch.cuda.Stream]] = {}


def lane_streams(device: torch.device, count: int) -> list[torch.cuda.Stream]:
    """The first `count` lane streams of `device`, created once per process
    and shared by every pipeline on the device (streams share the process's
    few hardware queues; a fresh set per pipeline could put two lanes on one
    queue and serialise them)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    with _stream_lock:
        lanes = _lanes.setdefault(index, [])
        while len(lanes) < count:
            lanes.append(torch.cuda.Stream(torch.device("cuda", index)))
        return lanes[:count]


def order_lanes_after(stream: torch.cuda.Stream, count: int) -> None:
    """Makes the first `count` lane streams of `stream`'s device wait for the
    work queued on `stream` so far.  The reference restores on the calling
    thread's current stream (worker.py:1087-1248), after everything queued
    there before; a restore issued after this call is ordered the same way
    (for instance after kernels of an earlier step that still read the
    blocks it overwrites)."""
    for lane in lane_streams(stream.device, max(2, int(count))):
        lane.wait_stream(stream)


class LayerRestorePipeline:
    """Copy-overlapped restore of one layer at a time into a cache, on
    `num_lanes` lane streams."""

    def __init__(self, device: torch.device | str, slot_bytes: int, num_lanes: int = 2,
                 host_staging: bool = True, grid_limit: int = 0,
                 staging_slots: int | None = None):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("LayerRestorePipeline needs a ROCm device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.slot_bytes = int(slot_bytes)
        self.lanes = lane_streams(self.device, max(2, int(num_lanes)))
        self._slots: list[torch.Tensor] = []
        for lane in self.lanes:
            dev = torch.empty(self.slot_bytes, dtype=torch.uint8, device=self.device)
            # written and read on the lane: its memory must outlive the work
            # queued there
            dev.record_stream(lane)
            self._slots.append(dev)
        n_staging = len(self.lanes) + 1 if staging_slots is None else max(1, int(staging_slots))
        self._staging = _StagingPool(n_staging, self.slot_bytes) if host_staging else None
        self._next = 0
        self._lock = threading.Lock()
        self._lane_last: list[torch.cuda.Event | None] = [None] * len(self.lanes)
        # Workgroup cap for the restore kernels: a restore hidden behind the
        # next layer's copy needs no more than a share of the GPU, and a
        # thinner launch leaves HBM bandwidth to the concurrent DMA.
        self.grid_limit = int(grid_limit)

    # -- internals ------------------------------------------------------------

    def _enqueue(self, src: torch.Tensor, nbytes: int, compute: Callable[[torch.Tensor], None],
                 timing: LayerTiming | None) -> tuple[torch.cuda.Event, torch.cuda.Event]:
        with self._lock:
            k = self._next % len(self.lanes)
            self._next += 1
            lane = self.lanes[k]
            flat = self._slots[k][:nbytes]
            copied, done = torch.cuda.Event(), torch.cuda.Event()
            with torch.cuda.stream(lane):
                if timing is not None:
                    timing.h2d_start.record(lane)
                flat.copy_(src[:nbytes], non_blocking=True)
                copied.record(lane)
                if timing is not None:
                    timing.h2d_end.record(lane)
                    timing.compute_start.record(lane)
                previous = _native.set_rows_grid_limit(self.grid_limit)
                try:
                    compute(flat)
                finally:
                    _native.set_rows_grid_limit(previous)
                if timing is not None:
                    timing.compute_end.record(lane)
                done.record(lane)
            self._lane_last[k] = done
            return done, copied

    # -- public API ----------------------------------------------------------

    def record_stream(self, tensor: torch.Tensor) -> None:
        """Marks a device tensor the restores read (e.g. a block table) as used
        on every lane."""
        for lane in self.lanes:
            tensor.record_stream(lane)

    def begin(self, stream: torch.cuda.Stream) -> None:
        """Makes every lane wait for the work queued so far on `stream` (a
        timing start, or inputs produced there)."""
        for lane in self.lanes:
            lane.wait_stream(stream)

    def join(self, stream: torch.cuda.Stream) -> None:
        """Makes `stream` wait for everything queued on the lanes so far."""
        for lane in self.lanes:
            stream.wait_stream(lane)

    def submit(self, source: torch.Tensor | Callable[[torch.Tensor], None], nbytes: int,
               compute: Callable[[torch.Tensor], None], *, timed: bool = False
               ) -> torch.cuda.Event | tuple[torch.cuda.Event, LayerTiming]:
        """One layer: bring `nbytes` of stream to the device and run `compute`
        on the device copy (on the layer's lane, after the copy).  `source` is
        either a pinned host tensor (copied directly; the caller keeps it alive
        until the returned event completes) or a callable that writes the
        stream into a pinned staging buffer.  The fill runs without any
        pipeline lock; the enqueue of one layer is never interleaved with
        another's.  With `timed`, returns (event, LayerTiming)."""
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
        """H2D of one stream into lane 0's slot with no compute: back-to-back
        calls are the bare copies the pipeline is measured against."""
        with self._lock:
            lane = self.lanes[0]
            done = torch.cuda.Event()
            with torch.cuda.stream(lane):
                self._slots[0][:nbytes].copy_(host_stream.reshape(-1)[:nbytes],
                                              non_blocking=True)
                done.record(lane)
            self._lane_last[0] = done
            return done

    def idle(self) -> bool:
        """True when every layer submitted so far has completed on the GPU."""
        with self._lock:
            last = list(self._lane_last)
        return all(e is None or e.query() for e in last)

    def synchronize(self) -> None:
        for lane in self.lanes:
            lane.synchronize()


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

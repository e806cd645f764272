"""Layer-wise restore pipeline on HIP streams and events.

Replaces the reference's same-stream restore (worker.py:1087-1248 issues the
H2D copies and the unpack/scatter on the worker thread's current stream, so
the copy of layer L+1 waits behind the unpack of layer L) with:

  host stream bytes (pinned)  --H2D, copy stream-->  device slot
      --fused unpack+scatter, compute stream-->  paged KV cache  --> event

* Device slots form a ring; a slot is refilled only after the unpack that
  read it has finished (compute-done event, waited on by the copy stream).
* Host data already in pinned memory is copied directly (the QAT path of the
  reference decompresses into pinned staging, native_cpu.py:307-316).  Other
  host data is first written into a pinned staging slot of the ring; a
  staging slot is reused only after its H2D copy has completed.
* Every layer gets its own completion event; wait_for_layer_load makes the
  attention stream wait on it (worker.py:553-572), so a layer's attention only
  depends on that layer.

All streams are created at the default priority.
"""
from __future__ import annotations

import threading
from dataclasses import dataclass
from typing import Callable

import torch

from origami_amd import _native
from origami_amd.layout import CanonicalLayout
from origami_amd.lossless import native_gpu


@dataclass
class _Slot:
    device: torch.Tensor
    host: torch.Tensor | None
    copy_done: torch.cuda.Event
    compute_done: torch.cuda.Event
    copy_recorded: bool = False
    compute_recorded: bool = False


class LayerRestorePipeline:
    """Copy/compute-overlapped restore of one layer at a time into a cache."""

    def __init__(self, device: torch.device | str, slot_bytes: int, num_slots: int = 3,
                 host_staging: bool = True, grid_limit: int = 0):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("LayerRestorePipeline needs a ROCm device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.slot_bytes = int(slot_bytes)
        self.copy_stream = torch.cuda.Stream(self.device)
        self.compute_stream = torch.cuda.Stream(self.device)
        self._slots: list[_Slot] = []
        for _ in range(max(2, int(num_slots))):
            dev = torch.empty(self.slot_bytes, dtype=torch.uint8, device=self.device)
            host = (torch.empty(self.slot_bytes, dtype=torch.uint8, pin_memory=True)
                    if host_staging else None)
            self._slots.append(_Slot(dev, host, torch.cuda.Event(), torch.cuda.Event()))
        self._next = 0
        self._lock = threading.Lock()
        # Workgroup cap for the restore kernels: a restore hidden behind the
        # next layer's copy needs no more than a share of the GPU, and a
        # thinner launch leaves HBM bandwidth to the concurrent DMA.
        self.grid_limit = int(grid_limit)

    # -- internals -----------------------------------------------------------

    def _h2d(self, slot: _Slot, src: torch.Tensor, nbytes: int) -> torch.Tensor:
        dst = slot.device[:nbytes]
        with torch.cuda.stream(self.copy_stream):
            if slot.compute_recorded:
                self.copy_stream.wait_event(slot.compute_done)  # device slot free
            dst.copy_(src[:nbytes], non_blocking=True)
            slot.copy_done.record(self.copy_stream)
            slot.copy_recorded = True
        return dst

    def _compute(self, slot: _Slot, flat: torch.Tensor,
                 compute: Callable[[torch.Tensor], None]) -> torch.cuda.Event:
        done = torch.cuda.Event()
        with torch.cuda.stream(self.compute_stream):
            self.compute_stream.wait_event(slot.copy_done)
            previous = _native.set_rows_grid_limit(self.grid_limit)
            try:
                compute(flat)
            finally:
                _native.set_rows_grid_limit(previous)
            slot.compute_done.record(self.compute_stream)
            slot.compute_recorded = True
            done.record(self.compute_stream)
        return done

    # -- public API ----------------------------------------------------------

    def submit(self, source: torch.Tensor | Callable[[torch.Tensor], None], nbytes: int,
               compute: Callable[[torch.Tensor], None]) -> torch.cuda.Event:
        """One layer: bring `nbytes` of stream to the device and run `compute`
        on the device copy (on the compute stream).  `source` is either a
        pinned host tensor (copied directly; the caller keeps it alive until
        the returned event completes) or a callable that writes the stream into
        a pinned staging buffer.  Calls are serialised: one layer's enqueue
        order is never interleaved with another's."""
        nbytes = int(nbytes)
        if nbytes > self.slot_bytes:
            raise RuntimeError("layer stream larger than the pipeline slot")
        with self._lock:
            slot = self._slots[self._next % len(self._slots)]
            self._next += 1
            if callable(source):
                if slot.host is None:
                    raise RuntimeError("pipeline was built without host staging")
                if slot.copy_recorded:
                    slot.copy_done.synchronize()  # previous H2D from this staging slot done
                staging = slot.host[:nbytes]
                source(staging)
                src = staging
            else:
                if source.numel() < nbytes:
                    raise RuntimeError("host stream shorter than the layer stream")
                src = source.reshape(-1)
            flat = self._h2d(slot, src, nbytes)
            return self._compute(slot, flat, compute)

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
            self._h2d(slot, host_stream.reshape(-1), nbytes)
            done = torch.cuda.Event()
            done.record(self.copy_stream)
            return done

    def synchronize(self) -> None:
        self.copy_stream.synchronize()
        self.compute_stream.synchronize()

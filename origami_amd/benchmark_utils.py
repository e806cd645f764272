"""Paged-cache scatter helper, tracing ranges and JSONL metrics.

copy_kv_to_hbm keeps the reference's signature and return values
(benchmark_utils.py:465-532): it normalises a restored K/V value to whole
blocks (zero-padding the tail, :350-432) and writes it into the paged cache
through the block table.  The write is the HIP block scatter of
liborigami_layout.so instead of index_copy_, and a value already in pinned
host memory is copied without blocking.  Metric fields named *_gbps are
gigabits per second, as in the reference.
"""
from __future__ import annotations

import json
import time
from contextlib import contextmanager
from dataclasses import asdict, dataclass
from pathlib import Path
from threading import Lock
from typing import Iterable

import torch

from origami_amd.lossless import native_gpu

_JSONL_LOCK = Lock()


@contextmanager
def nvtx_range(name: str):
    """A roctx range on ROCm (torch.cuda.nvtx maps to roctx)."""
    pushed = False
    if torch.cuda.is_available():
        try:
            torch.cuda.nvtx.range_push(name)
            pushed = True
        except Exception:  # noqa: BLE001 - tracing must never break the path
            pushed = False
    try:
        yield
    finally:
        if pushed:
            torch.cuda.nvtx.range_pop()


def write_jsonl(path: str | Path | None, record: dict) -> None:
    if not path:
        return
    p = Path(path)
    p.parent.mkdir(parents=True, exist_ok=True)
    with _JSONL_LOCK, p.open("a") as f:
        f.write(json.dumps(record, default=str) + "\n")


@dataclass
class H2DMetric:
    request_id: str
    cache_key: str
    system: str
    layer_name: str
    bytes_copied: int
    h2d_ms: float
    h2d_gbps: float
    start_ts: float
    end_ts: float
    device: str
    source_device: str
    copy_kind: str
    timing_complete: bool


def tensor_nbytes(tensor: torch.Tensor) -> int:
    return int(tensor.numel() * tensor.element_size())


def normalize_kv_value(kv_cache: torch.Tensor, block_count: int,
                       value: torch.Tensor) -> torch.Tensor:
    """Token-major [2, T, H, D] view of a restored value, for a cache of
    [2, NB, bs, H, D] or [NB, 2, bs, H, D] (the shapes _normalize_kv_value
    accepts: [2, nblk, bs, H, D], [nblk, 2, bs, H, D], [2, T, H, D], [2, H, T, D]).
    Tokens beyond block_count * bs are dropped."""
    bs, H, D = (int(x) for x in kv_cache.shape[2:])  # same in both cache layouts
    if value.dim() == 5:
        if value.shape[0] == 2 and value.shape[2] == bs and value.shape[3:] == (H, D):
            tok = value.reshape(2, -1, H, D)
        elif value.shape[1] == 2 and value.shape[2] == bs and value.shape[3:] == (H, D):
            tok = value.permute(1, 0, 2, 3, 4).reshape(2, -1, H, D)
        else:
            raise ValueError(f"Unsupported KV block value shape {tuple(value.shape)} "
                             f"for cache {tuple(kv_cache.shape)}")
    elif value.dim() == 4 and value.shape[0] == 2:
        if value.shape[2] == H and value.shape[3] == D:
            tok = value
        elif value.shape[1] == H and value.shape[3] == D:
            tok = value.permute(0, 2, 1, 3)
        else:
            raise ValueError("Unsupported HF KV artifact layer shape "
                             f"{tuple(value.shape)} for cache {tuple(kv_cache.shape)}")
    else:
        raise ValueError(f"Unsupported KV value shape {tuple(value.shape)}")
    needed = block_count * bs
    if tok.shape[1] > needed:
        tok = tok[:, :needed]
    return tok.contiguous()


def copy_kv_to_hbm(*, kv_cache: torch.Tensor, block_ids: Iterable[int], value: torch.Tensor,
                   request_id: str, cache_key: str, system: str, layer_name: str,
                   metrics_path: str | Path | None = None, synchronize: bool = True,
                   return_event: bool = False):
    if kv_cache.device.type != "cuda":
        raise RuntimeError("copy_kv_to_hbm writes a device KV cache; kv_cache is on the CPU")
    ids = block_ids if isinstance(block_ids, torch.Tensor) else [int(b) for b in block_ids]
    nblk = int(ids.numel()) if isinstance(ids, torch.Tensor) else len(ids)
    _, nb, bs, H, head_bytes = native_gpu.cache_geometry(kv_cache)
    source_device = str(value.device)
    bytes_copied = tensor_nbytes(value)
    start_ts = time.time()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with nvtx_range(f"{system}:h2d_copy"):
        start.record()
        tok = normalize_kv_value(kv_cache, nblk, value)
        if tok.device != kv_cache.device or tok.dtype != kv_cache.dtype:
            tok = tok.to(device=kv_cache.device, dtype=kv_cache.dtype,
                         non_blocking=bool(tok.device.type == "cpu" and tok.is_pinned()))
        ids_dev = native_gpu.block_ids_tensor(ids, kv_cache.device, nb)
        native_gpu.scatter_kv_blocks(tok, int(tok.shape[1]), kv_cache, ids_dev)
        end.record()
        if synchronize:
            end.synchronize()
    h2d_ms = float(start.elapsed_time(end)) if synchronize else 0.0
    metric = H2DMetric(
        request_id=request_id, cache_key=cache_key, system=system, layer_name=layer_name,
        bytes_copied=bytes_copied, h2d_ms=h2d_ms,
        h2d_gbps=(bytes_copied * 8.0 / h2d_ms / 1e6) if h2d_ms > 0 else 0.0,
        start_ts=start_ts, end_ts=time.time(), device=str(kv_cache.device),
        source_device=source_device,
        copy_kind="hbm_to_hbm" if source_device.startswith("cuda") else "dram_to_hbm",
        timing_complete=bool(synchronize),
    )
    write_jsonl(metrics_path, {"type": "h2d_copy", **asdict(metric)})
    if return_event:
        return metric, end
    return metric

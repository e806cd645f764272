"""GPU layout path: Python front end of liborigami_layout.so.

Mirrors lossless/native_gpu.py of the reference (load_bitpack_cuda_extension,
available, unpack_canonical_storage_chunks, cachegen_unpack_dequantize*,
kivi_dequantize_to_kv_cache; native_gpu.py:35-261) and adds the pieces the reference lacks: the pack, the
fused unpack+scatter into the paged KV cache and the fused gather+pack from
it.

All work is enqueued on the calling thread's current stream of the tensors'
device, like the reference (bitpack_layout_cuda.cpp:370).  Chunk metadata stays
on the host: no call reads device memory back.
"""
from __future__ import annotations

import contextlib
import ctypes
import functools
from functools import lru_cache
from typing import Iterable, Sequence

import numpy as np
import torch

from origami_amd import _ext, _native
from origami_amd.layout import CanonicalLayout, kv_symbol_layout

CACHE_KV_FIRST = _native.CACHE_KV_FIRST
CACHE_BLOCKS_FIRST = _native.CACHE_BLOCKS_FIRST


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle(device: torch.device):
    """The calling thread's current stream on `device`, as a raw handle."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return ctypes.c_void_p(_raw_stream(index))
    return ctypes.c_void_p(torch.cuda.current_stream(index).cuda_stream)


def _device_guard(device: torch.device):
    """Makes `device` current for the call (a no-op when it already is)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


def _require_cuda(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def available() -> bool:
    """True when a GPU is visible and the native library loads."""
    if not torch.cuda.is_available():
        return False
    try:
        _native.lib()
        _ext.ext()
        return True
    except Exception:  # noqa: BLE001 - mirrors the reference's available()
        return False


# ---------------------------------------------------------------------------
# Flat streams
# ---------------------------------------------------------------------------

def flat_chunks_and_offsets(chunks: Iterable[torch.Tensor] | torch.Tensor,
                            device: torch.device) -> tuple[torch.Tensor, list[int]]:
    """Concatenates chunk tensors on `device` (native_gpu.py:92-110)."""
    if isinstance(chunks, torch.Tensor):
        flat = chunks.detach().reshape(-1)
        if flat.device != device or flat.dtype != torch.uint8:
            flat = flat.to(device=device, dtype=torch.uint8, non_blocking=True)
        return flat.contiguous(), [0, int(flat.numel())]
    parts, offsets, total = [], [0], 0
    for chunk in chunks:
        part = chunk.detach().reshape(-1).to(device=device, dtype=torch.uint8, non_blocking=True)
        parts.append(part)
        total += int(part.numel())
        offsets.append(total)
    if not parts:
        return torch.empty((0,), dtype=torch.uint8, device=device), offsets
    flat = parts[0] if len(parts) == 1 else torch.cat(parts)
    return flat.contiguous(), offsets


def _layout_args(layout: CanonicalLayout) -> tuple:
    return layout.native_args


# ---------------------------------------------------------------------------
# Canonical pack / unpack (source-layout symbol tensors)
# ---------------------------------------------------------------------------

def unpack_layout(flat: torch.Tensor, layout: CanonicalLayout,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """Unpacks a flat stream into a new (or given) uint8 symbol tensor."""
    _require_cuda(flat, "flat_chunks")
    if flat.dtype != torch.uint8:
        raise RuntimeError("flat_chunks must be uint8")
    if out is None:
        offs, bits, specs = layout.torch_meta
        shape, axes = layout.torch_shape_axes
        return _ext.ext().unpack_canonical_storage_chunks_cuda(
            flat, offs, bits, shape, axes, layout.token_count, layout.num_heads,
            layout.head_dim, specs)
    _require_cuda(out, "output")
    with _device_guard(flat.device):
        _native.call(
            "origami_unpack_canonical_storage_chunks",
            flat.data_ptr(), flat.numel(), *_layout_args(layout),
            _native.host_ptr(layout.shape_arr), len(layout.shape), _native.host_ptr(layout.axes),
            layout.token_count, layout.num_heads, layout.head_dim,
            out.data_ptr(), out.numel(), _stream_handle(flat.device))
    return out


def pack_layout(symbols: torch.Tensor, layout: CanonicalLayout,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """Packs a uint8 symbol tensor into a new (or given) flat stream."""
    _require_cuda(symbols, "symbols")
    if symbols.dtype != torch.uint8:
        raise RuntimeError("symbols must be uint8")
    if out is None:
        out = torch.empty((layout.stream_bytes,), dtype=torch.uint8, device=symbols.device)
    shape, axes = layout.torch_shape_axes
    _ext.ext().pack_canonical_storage_chunks(symbols, *layout.torch_meta, shape, axes,
                                             layout.token_count, layout.num_heads,
                                             layout.head_dim, out)
    return out


def unpack_canonical_storage_chunks(
    chunks: Iterable[torch.Tensor] | torch.Tensor,
    bits: int | Sequence[int],
    source_shape: Sequence[int],
    source_layout: Sequence[str],
    chunk_specs,
    *,
    device: torch.device | str | None = None,
) -> torch.Tensor:
    """Same contract as the reference (native_gpu.py:113-146): returns the
    flat uint8 symbol tensor of prod(source_shape) bytes on `device`."""
    target = torch.device(device or "cuda")
    if target.type == "cuda" and target.index is None:
        target = torch.device("cuda", torch.cuda.current_device())
    layout = CanonicalLayout.make(source_shape, source_layout, bits, chunk_specs)
    flat, offsets = flat_chunks_and_offsets(chunks, target)
    if not isinstance(chunks, torch.Tensor) and len(offsets) - 1 != layout.num_chunks:
        raise RuntimeError("Origami native layout metadata chunk count does not match payload chunks")
    if not isinstance(chunks, torch.Tensor) and not np.array_equal(
            np.asarray(offsets, dtype=np.int64), layout.offsets):
        raise RuntimeError("Origami CUDA packed chunk byte size mismatch")
    return unpack_layout(flat, layout)


def pack_canonical_storage_flat(
    symbols: torch.Tensor,
    bits: int | Sequence[int],
    source_shape: Sequence[int],
    source_layout: Sequence[str],
    chunk_specs,
) -> tuple[torch.Tensor, CanonicalLayout]:
    """Packs on the symbols' device; returns (flat stream, layout)."""
    layout = CanonicalLayout.make(source_shape, source_layout, bits, chunk_specs)
    flat_symbols = symbols.detach().reshape(-1)
    if flat_symbols.dtype != torch.uint8:
        flat_symbols = flat_symbols.to(torch.uint8)
    return pack_layout(flat_symbols.contiguous(), layout), layout


def pack_canonical_storage_chunks(
    symbols: torch.Tensor,
    bits: int | Sequence[int],
    source_shape: Sequence[int],
    source_layout: Sequence[str],
    chunk_specs,
) -> list[torch.Tensor]:
    """The packer the reference leaves as a stub (native_cpu.py:144-151):
    returns one uint8 tensor per chunk spec (views of one device stream)."""
    flat, layout = pack_canonical_storage_flat(symbols, bits, source_shape, source_layout,
                                               chunk_specs)
    off = layout.offsets
    return [flat[int(off[k]):int(off[k + 1])] for k in range(layout.num_chunks)]


# ---------------------------------------------------------------------------
# Paged KV cache
# ---------------------------------------------------------------------------

def cache_geometry(kv_cache: torch.Tensor, num_heads: int | None = None,
                   head_dim: int | None = None) -> tuple[int, int, int, int, int]:
    """(layout code, num_blocks, block_size, heads, head_bytes) of a rank-5
    paged cache.  [2, NB, bs, H, D] is recognised first (the rule of
    benchmark_utils.py:357 and bitpack_layout_cuda.cpp:810-831), then
    [NB, 2, bs, H, D]."""
    if kv_cache.dim() != 5:
        raise RuntimeError("kv_cache must have rank 5")
    if kv_cache.shape[0] == 2:
        code, nb = CACHE_KV_FIRST, int(kv_cache.shape[1])
    elif kv_cache.shape[1] == 2:
        code, nb = CACHE_BLOCKS_FIRST, int(kv_cache.shape[0])
    else:
        raise RuntimeError("kv_cache must be [num_blocks,2,block,heads,dim] or "
                           "[2,num_blocks,block,heads,dim]")
    bs, H, D = (int(x) for x in kv_cache.shape[2:])
    if num_heads is not None and head_dim is not None and (H != num_heads or D != head_dim):
        raise RuntimeError("kv_cache head shape mismatch")
    return code, nb, bs, H, D * kv_cache.element_size()


def block_ids_tensor(block_ids, device: torch.device, num_blocks: int | None = None
                     ) -> torch.Tensor:
    """int64 device block table; ids are validated on the host first."""
    if isinstance(block_ids, torch.Tensor):
        ids_cpu = block_ids.detach().to("cpu", torch.int64)
    else:
        ids_cpu = torch.tensor([int(b) for b in block_ids], dtype=torch.int64)
    if ids_cpu.numel() == 0:
        raise RuntimeError("block_ids must be non-empty")
    if num_blocks is not None and (int(ids_cpu.min()) < 0 or int(ids_cpu.max()) >= num_blocks):
        raise RuntimeError("block id out of range for kv_cache")
    if isinstance(block_ids, torch.Tensor) and block_ids.device == device \
            and block_ids.dtype == torch.int64 and block_ids.is_contiguous():
        return block_ids
    return ids_cpu.to(device).contiguous()


def unpack_to_kv_cache(flat: torch.Tensor, layout: CanonicalLayout, tokens: int,
                       kv_cache: torch.Tensor, block_ids: torch.Tensor) -> None:
    """Fused restore of one layer: stream -> paged cache through the block
    table.  `layout` is the [2*tokens, H, head_bytes] symbol layout of the
    layer (kv_symbol_layout).  Falls back to unpack + scatter (both on the
    GPU) when the chunk plan is not served by the fused kernel."""
    if (layout.token_count != 2 * tokens or kv_cache.dim() != 5
            or layout.num_heads != kv_cache.shape[3]
            or layout.head_dim != kv_cache.shape[4] * kv_cache.element_size()):
        raise RuntimeError("symbol layout does not match the kv_cache geometry")
    if _ext.ext().unpack_canonical_to_kv_cache(flat, *layout.torch_meta, tokens, kv_cache,
                                               block_ids):
        return
    # Irregular chunk plan: unpack to the symbol tensor, then scatter.
    symbols = unpack_layout(flat, layout) if layout.layout == ("token", "head", "head_dim") \
        else _unpack_kv_tokens_major(flat, layout)
    scatter_kv_blocks(symbols, tokens, kv_cache, block_ids)


def _unpack_kv_tokens_major(flat: torch.Tensor, layout: CanonicalLayout) -> torch.Tensor:
    """Unpack in any source layout, then permute to token-major bytes."""
    sym = unpack_layout(flat, layout).reshape(layout.shape)
    order = [int(layout.axes[0]), int(layout.axes[1]), int(layout.axes[2])]
    if layout.axes[3] >= 0:
        sym = sym.squeeze(int(layout.axes[3]))
        order = [a - (1 if a > layout.axes[3] else 0) for a in order]
    return sym.permute(*order).contiguous().reshape(-1)


def pack_from_kv_cache(kv_cache: torch.Tensor, block_ids: torch.Tensor, tokens: int,
                       layout: CanonicalLayout, out: torch.Tensor | None = None) -> torch.Tensor:
    """Fused save of one layer: paged cache -> stream.  Falls back to gather +
    pack (both on the GPU) when the plan is not served by the fused kernel."""
    _require_cuda(kv_cache, "kv_cache")
    code, nb, bs, H, head_bytes = cache_geometry(kv_cache)
    if layout.token_count != 2 * tokens or layout.num_heads != H or layout.head_dim != head_bytes:
        raise RuntimeError("symbol layout does not match the kv_cache geometry")
    if out is None:
        out = torch.empty((layout.stream_bytes,), dtype=torch.uint8, device=kv_cache.device)
    if _ext.ext().pack_canonical_from_kv_cache(kv_cache, block_ids, int(tokens),
                                               *layout.torch_meta, out):
        return out
    value = gather_kv_blocks(kv_cache, block_ids)
    nblk_tokens = block_ids.numel() * bs
    value = value.reshape(2, nblk_tokens, H * head_bytes)[:, :tokens].contiguous()
    if layout.layout != ("token", "head", "head_dim"):
        value = _tokens_major_to_layout(value.reshape(-1), layout)
    return pack_layout(value.reshape(-1), layout, out)


def _tokens_major_to_layout(value: torch.Tensor, layout: CanonicalLayout) -> torch.Tensor:
    T, H, C = layout.token_count, layout.num_heads, layout.head_dim
    tmaj = value.reshape(T, H, C)
    names = [n for n in layout.layout if n != "layer"]
    src = {"token": 0, "head": 1, "head_dim": 2}
    out = tmaj.permute(*[src[n] for n in names]).contiguous()
    return out.reshape(-1)


def batch_block_tables(block_tables: Sequence, tokens: Sequence[int], block_size: int,
                       dedup: bool) -> tuple[list[np.ndarray], bool]:
    """Host block tables of a batched restore, and whether the requests may
    share one launch.  A destination block that several requests restore as a
    full block (all block_size tokens valid) holds the same bytes in each
    (vLLM shares only full prefix blocks); with `dedup` its later occurrences
    become -1, so it is read and written once.  A block that is partial in any
    request that shares it would receive different bytes, so such a batch
    must run request by request (returned flag False)."""
    tables = [np.ascontiguousarray(np.asarray(t, dtype=np.int64).reshape(-1))
              for t in block_tables]
    if len(tables) < 2:
        return tables, True
    full = [np.arange(1, t.size + 1) * block_size <= int(T) for t, T in zip(tables, tokens)]
    cat = np.concatenate(tables)
    fcat = np.concatenate(full)
    uniq, first = np.unique(cat, return_index=True)
    first_of = first[np.searchsorted(uniq, cat)]
    dup = np.arange(cat.size) != first_of
    if not dup.any():
        return tables, True
    if (dup & ~(fcat & fcat[first_of])).any():
        return tables, False
    if dedup:
        cat = cat.copy()
        cat[dup] = -1
        bounds = np.cumsum([0] + [t.size for t in tables])
        tables = [cat[bounds[i]:bounds[i + 1]] for i in range(len(tables))]
    return tables, True


class KVRestoreBatch:
    """One layer of several requests restored into a cache per call, the
    block tables prepared once for all layers of the batch.  The reference
    restores request by request (worker.py:796-897 and 1087-1248); here each
    layer is one native call and one launch per symbol width and addressing
    mode.  `layouts[r]`, `tokens[r]` and `block_tables[r]` (host ids) describe
    request r; the result of restore() equals restoring the requests one
    after another.  With `dedup_shared_blocks` a full block shared by several
    requests (vLLM prefix blocks hold the same bytes) is written once, from the
    first request that has it; a later request's leading shared blocks are
    not read either."""

    def __init__(self, layouts: Sequence[CanonicalLayout], tokens: Sequence[int],
                 block_tables: Sequence, kv_cache: torch.Tensor, *,
                 dedup_shared_blocks: bool = False):
        _require_cuda(kv_cache, "kv_cache")
        self.geometry = cache_geometry(kv_cache)
        self.device = kv_cache.device
        self._shape, self._dtype = tuple(kv_cache.shape), kv_cache.dtype
        code, nb, bs, H, head_bytes = self.geometry
        self.layouts = list(layouts)
        self.tokens = [int(t) for t in tokens]
        if not (len(self.layouts) == len(self.tokens) == len(block_tables)):
            raise RuntimeError("layouts, tokens and block tables must have one entry per request")
        for layout, T in zip(self.layouts, self.tokens):
            if (layout.token_count != 2 * T or layout.num_heads != H
                    or layout.head_dim != head_bytes):
                raise RuntimeError("symbol layout does not match the kv_cache geometry")
        host = []
        for ids in block_tables:
            ids_np = (ids.detach().to("cpu", torch.int64).numpy()
                      if isinstance(ids, torch.Tensor) else np.asarray(ids, dtype=np.int64))
            ids_np = ids_np.reshape(-1)
            if ids_np.size == 0:
                raise RuntimeError("block_ids must be non-empty")
            if int(ids_np.min()) < 0 or int(ids_np.max()) >= nb:
                raise RuntimeError("block id out of range for kv_cache")
            host.append(ids_np)
        dedup = bool(dedup_shared_blocks) and bs % 16 == 0
        tables, self.batchable = batch_block_tables(host, self.tokens, bs, dedup)
        # a request's leading shared blocks are not read or written at all
        # (its restore starts past them); other shared blocks are skipped on
        # write (ids -1)
        lead = []
        for t in tables:
            live = np.flatnonzero(t >= 0)
            lead.append(int(live[0]) if live.size else int(t.size))
        self.skipped_blocks = int(sum(lead))
        self._first = np.ascontiguousarray(np.asarray([k * bs for k in lead], dtype=np.int64))
        self.block_counts = [int(t.size) for t in tables]
        n = len(tables)
        if n:
            self._dev_tables = torch.from_numpy(np.concatenate(tables)).to(self.device)
        bounds = np.cumsum([0] + self.block_counts)
        self.tables = [self._dev_tables[int(bounds[i]):int(bounds[i + 1])] for i in range(n)]
        self._offs = [lay.torch_meta[0] for lay in self.layouts]
        self._bits = [lay.torch_meta[1] for lay in self.layouts]
        self._specs = [lay.torch_meta[2] for lay in self.layouts]
        self._first_list = [int(x) for x in self._first]

    def record_stream(self, stream: torch.cuda.Stream) -> None:
        """Marks the device block tables as used on `stream` (restores queued
        there keep them alive after this object is dropped)."""
        if self.layouts:
            self._dev_tables.record_stream(stream)

    def restore(self, flats: Sequence[torch.Tensor], kv_cache: torch.Tensor) -> None:
        """Restores one layer: flats[r] is request r's stream on the device."""
        if len(flats) != len(self.layouts):
            raise RuntimeError("one stream per request is required")
        if tuple(kv_cache.shape) != self._shape or kv_cache.dtype != self._dtype \
                or kv_cache.device != self.device:
            raise RuntimeError("kv_cache geometry differs from the prepared batch")
        if not self.layouts:
            return
        if not self.batchable:
            for flat, layout, T, ids in zip(flats, self.layouts, self.tokens, self.tables):
                unpack_to_kv_cache(flat, layout, T, kv_cache, ids)
            return
        if _ext.ext().unpack_canonical_to_kv_cache_batch(
                list(flats), self._offs, self._bits, self._specs, self.tokens, kv_cache,
                self.tables, self._first_list):
            return
        for flat, layout, T, ids in zip(flats, self.layouts, self.tokens, self.tables):
            unpack_to_kv_cache(flat, layout, T, kv_cache, ids)  # irregular plans


class PreparedRestore:
    """The fused restore of one request prepared once for all of its layers:
    the chunk plan, tokens, cache geometry and block table are checked and
    looked up at construction, and restore(flat, kv_cache) then launches with
    only the layer's stream and destination cache (origami_restore_plan_*).
    The reference restores each layer through the full extension call
    (worker.py:1087-1248); results equal unpack_to_kv_cache's.  `supported` is
    False when the chunk plan is not served by the fused kernel; restore() then
    takes unpack_to_kv_cache's two-step path.  Every kv_cache passed to
    restore() must have the shape, dtype and device of the one given here."""

    def __init__(self, layout: CanonicalLayout, tokens: int, kv_cache: torch.Tensor,
                 block_ids):
        _require_cuda(kv_cache, "kv_cache")
        if (layout.token_count != 2 * tokens or kv_cache.dim() != 5
                or layout.num_heads != kv_cache.shape[3]
                or layout.head_dim != kv_cache.shape[4] * kv_cache.element_size()):
            raise RuntimeError("symbol layout does not match the kv_cache geometry")
        self.layout, self.tokens = layout, int(tokens)
        self.block_ids = block_ids_tensor(block_ids, kv_cache.device,
                                          cache_geometry(kv_cache)[1])
        self._ext = _ext.ext()
        self._handle = int(self._ext.restore_plan_create(*layout.torch_meta, self.tokens,
                                                         kv_cache, self.block_ids))
        self.supported = self._handle != 0
        if self.supported:
            # restore(flat, kv_cache) is the extension call itself: no Python
            # frame of its own between the caller and the launch
            self.restore = functools.partial(self._ext.restore_plan_launch, self._handle)

    def restore(self, flat: torch.Tensor, kv_cache: torch.Tensor) -> None:
        """Restores one layer's stream `flat` into `kv_cache` on the current stream."""
        if self.supported:
            raise RuntimeError("restore plan is closed")
        unpack_to_kv_cache(flat, self.layout, self.tokens, kv_cache, self.block_ids)

    def close(self) -> None:
        """Frees the plan (work already enqueued keeps nothing of it)."""
        h, self._handle = self._handle, 0
        self.__dict__.pop("restore", None)  # restore() now raises
        if h:
            self._ext.restore_plan_destroy(h)

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown
            pass


def unpack_batch_to_kv_cache(requests: Sequence[tuple], kv_cache: torch.Tensor, *,
                             dedup_shared_blocks: bool = False) -> None:
    """One layer of several requests, (flat stream, kv_symbol_layout, tokens,
    host block ids) each, restored into one cache (KVRestoreBatch for a
    single layer)."""
    reqs = list(requests)
    batch = KVRestoreBatch([r[1] for r in reqs], [r[2] for r in reqs], [r[3] for r in reqs],
                           kv_cache, dedup_shared_blocks=dedup_shared_blocks)
    batch.restore([r[0] for r in reqs], kv_cache)


def scatter_kv_blocks(value: torch.Tensor, tokens: int, kv_cache: torch.Tensor,
                      block_ids: torch.Tensor) -> None:
    """Token-major K/V bytes [2, tokens, H, head_bytes] -> paged cache,
    zero-padding the last block (benchmark_utils.py:350-444)."""
    _require_cuda(value, "value")
    _require_cuda(kv_cache, "kv_cache")
    _require_cuda(block_ids, "block_ids")
    code, nb, bs, H, head_bytes = cache_geometry(kv_cache)
    if value.numel() * value.element_size() != 2 * tokens * H * head_bytes:
        raise RuntimeError("value size does not match 2 * tokens * heads * head_dim")
    with _device_guard(kv_cache.device):
        _native.call("origami_scatter_kv_blocks", value.data_ptr(), int(tokens),
                     kv_cache.data_ptr(), code, nb, bs, H, head_bytes,
                     block_ids.data_ptr(), block_ids.numel(), _stream_handle(kv_cache.device))


def gather_kv_blocks(kv_cache: torch.Tensor, block_ids: torch.Tensor,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """Paged cache -> token-major bytes [2, nblk*bs, H, head_bytes] (uint8)."""
    _require_cuda(kv_cache, "kv_cache")
    _require_cuda(block_ids, "block_ids")
    code, nb, bs, H, head_bytes = cache_geometry(kv_cache)
    n = 2 * block_ids.numel() * bs * H * head_bytes
    if out is None:
        out = torch.empty((n,), dtype=torch.uint8, device=kv_cache.device)
    with _device_guard(kv_cache.device):
        _native.call("origami_gather_kv_blocks", kv_cache.data_ptr(), code, nb, bs, H,
                     head_bytes, block_ids.data_ptr(), block_ids.numel(), out.data_ptr(),
                     _stream_handle(kv_cache.device))
    return out


# ---------------------------------------------------------------------------
# Fused dequantize paths (CacheGen, KIVI)
# ---------------------------------------------------------------------------

_DTYPE_CODES = {
    torch.float16: _native.DTYPE_FLOAT16,
    torch.bfloat16: _native.DTYPE_BFLOAT16,
    torch.float32: _native.DTYPE_FLOAT32,
}


def dequant_cache_geometry(kv_cache: torch.Tensor, heads: int, head_dim: int
                           ) -> tuple[int, int, int]:
    """(layout code, num_blocks, block_size) for the fused dequantize paths.
    These follow bitpack_layout_cuda.cpp:526-552, which recognises
    [NB, 2, bs, H, D] first and [2, NB, bs, H, D] second (the opposite
    order from cache_geometry)."""
    if kv_cache.dim() != 5:
        raise RuntimeError("kv_cache must have rank 5")
    if int(kv_cache.shape[1]) == 2:
        code, nb = CACHE_BLOCKS_FIRST, int(kv_cache.shape[0])
    elif int(kv_cache.shape[0]) == 2:
        code, nb = CACHE_KV_FIRST, int(kv_cache.shape[1])
    else:
        raise RuntimeError("kv_cache must be [num_blocks,2,block,heads,dim] or "
                           "[2,num_blocks,block,heads,dim]")
    if int(kv_cache.shape[3]) != int(heads) or int(kv_cache.shape[4]) != int(head_dim):
        raise RuntimeError("kv_cache head shape mismatch")
    return code, nb, int(kv_cache.shape[2])


def _max_tensors(max_key: torch.Tensor, max_value: torch.Tensor) -> int:
    _require_cuda(max_key, "max_key")
    _require_cuda(max_value, "max_value")
    if max_key.dtype != max_value.dtype:
        raise RuntimeError("max_key and max_value must have the same dtype")
    if max_key.dtype not in (torch.float16, torch.float32):
        raise RuntimeError("max tensors must be float16 or float32")
    return _DTYPE_CODES[max_key.dtype]


def cachegen_unpack_dequantize_to_kv_cache(
    bytestream: torch.Tensor, *, key_offset: int, key_bytes: int, value_offset: int,
    value_bytes: int, key_bits: int, value_bits: int, key_bins: int, value_bins: int,
    max_key: torch.Tensor, max_value: torch.Tensor, kv_cache: torch.Tensor,
    block_ids: torch.Tensor, tokens: int, heads: int, head_dim: int,
) -> None:
    """CacheGen fused restore into the paged cache (native_gpu.py:178-215,
    bitpack_layout_cuda.cpp:475-581): the K and V streams are unpacked,
    dequantized ((s - c) / c * max[token]) and written to the listed blocks
    in one kernel per half.  Tokens >= `tokens` are left untouched."""
    flat = bytestream.reshape(-1)
    if not flat.is_contiguous():
        flat = flat.contiguous()
    _require_cuda(flat, "bytestream")
    if flat.dtype != torch.uint8:
        raise RuntimeError("bytestream must be uint8")
    _require_cuda(kv_cache, "kv_cache")
    if kv_cache.dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError("kv_cache must be float16 or bfloat16")
    max_key, max_value = max_key.contiguous(), max_value.contiguous()
    _max_tensors(max_key, max_value)
    ids = block_ids.to(device=kv_cache.device, dtype=torch.int64).contiguous()
    dequant_cache_geometry(kv_cache, heads, head_dim)
    _ext.ext().cachegen_unpack_dequantize_to_kv_cache_cuda(
        flat, int(key_offset), int(key_bytes), int(value_offset), int(value_bytes),
        int(key_bits), int(value_bits), int(key_bins), int(value_bins), max_key, max_value,
        kv_cache, ids, int(tokens), int(heads), int(head_dim))


def _host_i64(values) -> np.ndarray:
    if isinstance(values, torch.Tensor):
        values = values.detach().to("cpu", torch.int64).reshape(-1).numpy()
    return _native.i64_array(values)


def cachegen_unpack_dequantize(
    bytestream: torch.Tensor, offsets, bits_per_layer, key_bins, value_bins,
    max_key: torch.Tensor, max_value: torch.Tensor, *, tokens: int, heads: int, head_dim: int,
) -> torch.Tensor:
    """CacheGen unpack + dequantize of `layers` layers into a float16 tensor
    [layers, 2, heads, tokens, head_dim] (native_gpu.py:149-175,
    bitpack_layout_cuda.cpp:402-473).  Stream segment j of `offsets` is
    layer j's keys for j < layers and layer j - layers' values after that."""
    flat = bytestream.reshape(-1)
    if not flat.is_contiguous():
        flat = flat.contiguous()
    _require_cuda(flat, "bytestream")
    if flat.dtype != torch.uint8:
        raise RuntimeError("bytestream must be uint8")
    offs, bits = _host_i64(offsets), _host_i64(bits_per_layer)
    kb, vb = _host_i64(key_bins), _host_i64(value_bins)
    if bits.size % 2:
        raise RuntimeError("bits_per_layer length must be even")
    layers = bits.size // 2
    if kb.size != layers:
        raise RuntimeError("key_bins length must match layers")
    if vb.size != layers:
        raise RuntimeError("value_bins length must match layers")
    if offs.size != bits.size + 1:
        raise RuntimeError("offsets length must be bits_per_layer length + 1")
    max_key, max_value = max_key.contiguous(), max_value.contiguous()
    _max_tensors(max_key, max_value)
    return _ext.ext().cachegen_unpack_dequantize_cuda(
        flat, torch.from_numpy(offs), torch.from_numpy(bits), torch.from_numpy(kb),
        torch.from_numpy(vb), max_key, max_value, int(tokens), int(heads), int(head_dim))


_KIVI_PACKING = {"lsb": _native.KIVI_PACKED_LSB, "kivi": _native.KIVI_NIBBLE3}


def kivi_dequantize_to_kv_cache(
    bytestream: torch.Tensor, *, key_offset: int, key_bytes: int, value_offset: int,
    value_bytes: int, bits: int, group_size: int, sink_tokens: int, key_scale: torch.Tensor,
    key_zero: torch.Tensor, value_scale: torch.Tensor, value_zero: torch.Tensor,
    key_sink: torch.Tensor, value_sink: torch.Tensor, kv_cache: torch.Tensor,
    block_ids: torch.Tensor, tokens: int, heads: int, head_dim: int,
    symbol_packing: str = "lsb",
) -> None:
    """KIVI fused restore into the paged cache (native_gpu.py:218-261,
    bitpack_layout_cuda.cpp:583-714): sink tokens are copied, body tokens
    dequantized with per-channel key groups and per-token value groups, all
    written through the block table.  symbol_packing "lsb" reads b-bit
    symbols LSB-first, as the reference kernel does; "kivi" reads KIVI's own
    container (kivi_adapter.py:28-54), whose 3-bit symbols sit one per
    nibble."""
    flat = bytestream.reshape(-1)
    if not flat.is_contiguous():
        flat = flat.contiguous()
    _require_cuda(flat, "bytestream")
    if flat.dtype != torch.uint8:
        raise RuntimeError("bytestream must be uint8")
    _require_cuda(kv_cache, "kv_cache")
    if kv_cache.dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError("kv_cache must be float16 or bfloat16")
    metas = [t.contiguous() for t in (key_scale, key_zero, value_scale, value_zero, key_sink,
                                      value_sink)]
    for t, name in zip(metas, ("key_scale", "key_zero", "value_scale", "value_zero", "key_sink",
                               "value_sink")):
        _require_cuda(t, name)
    if any(t.dtype != metas[0].dtype for t in metas):
        raise RuntimeError("KIVI metadata tensors must have the same dtype")
    if metas[0].dtype not in (torch.float16, torch.float32):
        raise RuntimeError("KIVI metadata tensors must be float16 or float32")
    if symbol_packing not in _KIVI_PACKING:
        raise ValueError(f"symbol_packing must be one of {sorted(_KIVI_PACKING)}")
    ids = block_ids.to(device=kv_cache.device, dtype=torch.int64).contiguous()
    dequant_cache_geometry(kv_cache, heads, head_dim)
    _ext.ext().kivi_dequantize_to_kv_cache(
        flat, int(key_offset), int(key_bytes), int(value_offset), int(value_bytes), int(bits),
        _KIVI_PACKING[symbol_packing], int(group_size), int(sink_tokens), *metas, kv_cache, ids,
        int(tokens), int(heads), int(head_dim))


# ---------------------------------------------------------------------------
# Reference extension surface (origami_bitpack_cuda_v6, cpp:894-903)
# ---------------------------------------------------------------------------

@lru_cache(maxsize=1)
def load_bitpack_cuda_extension():
    """Counterpart of native_gpu.load_bitpack_cuda_extension (py:35-49): the
    AOT-built PyTorch-ROCm module origami_bitpack_hip instead of a JIT-built
    CUDA extension.  It exports the reference module's functions
    (unpack_canonical_storage_chunks_cuda, cachegen_unpack_dequantize_cuda,
    cachegen_unpack_dequantize_to_kv_cache_cuda,
    kivi_dequantize_to_kv_cache_cuda, fused_prefix_attention_cuda) with their
    argument lists; chunk metadata may be host or device tensors (device
    ones cost one device-to-host copy each, as in the reference)."""
    if not torch.cuda.is_available():
        raise RuntimeError("Origami HIP layout library requires a ROCm GPU")
    return _ext.ext()


__all__ = [
    "available", "load_bitpack_cuda_extension", "flat_chunks_and_offsets",
    "unpack_canonical_storage_chunks", "pack_canonical_storage_chunks",
    "pack_canonical_storage_flat", "unpack_layout", "pack_layout", "cache_geometry",
    "block_ids_tensor", "unpack_to_kv_cache", "pack_from_kv_cache", "scatter_kv_blocks",
    "gather_kv_blocks", "kv_symbol_layout", "CACHE_KV_FIRST", "CACHE_BLOCKS_FIRST",
    "cachegen_unpack_dequantize_to_kv_cache", "cachegen_unpack_dequantize",
    "kivi_dequantize_to_kv_cache", "dequant_cache_geometry",
]

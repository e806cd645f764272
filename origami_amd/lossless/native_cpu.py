"""Host-side layout API (lossless/native_cpu.py:30-199 of the reference).

The reference ships this module's pack/unpack as stubs that raise
(native_cpu.py:137-161).  Here they work: they run on the GPU through
liborigami_layout.so and hand back CPU tensors, which is what the save path's
CPU codec consumes.  Without a ROCm GPU they raise, as there is no CPU
implementation in the product.  The QAT entry points of the reference module
are outside this build (host decompression stays with the CPU codec).
"""
from __future__ import annotations

from typing import Iterable, Sequence

import torch

from origami_amd.layout import (  # noqa: F401  (re-exported reference API)
    STORAGE_LAYOUT,
    _AXIS_ALIASES,
    axis_positions,
    canonical_axis_sizes,
    normalize_symbol_layout,
)
from origami_amd.lossless import native_gpu


def _gpu_device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError(
            "Origami layout packing runs on the GPU (liborigami_layout.so); "
            "no ROCm device is visible")
    return torch.device("cuda", torch.cuda.current_device())


def pack_canonical_storage_chunks(
    symbols: torch.Tensor,
    bits: int,
    source_shape: Sequence[int],
    source_layout: Sequence[str],
    chunk_specs,
) -> list[torch.Tensor]:
    """Returns one CPU uint8 tensor per chunk spec (ceil(n*b/8) bytes each)."""
    dev = symbols.device if symbols.is_cuda else _gpu_device()
    flat, layout = native_gpu.pack_canonical_storage_flat(
        symbols.detach().to(dev), bits, source_shape, source_layout, chunk_specs)
    host = flat.cpu()
    off = layout.offsets
    return [host[int(off[k]):int(off[k + 1])] for k in range(layout.num_chunks)]


def unpack_canonical_storage_chunks(
    chunks: Iterable[torch.Tensor],
    bits: int,
    source_shape: Sequence[int],
    source_layout: Sequence[str],
    chunk_specs,
) -> torch.Tensor:
    """Returns the flat CPU uint8 symbol tensor of prod(source_shape) bytes."""
    dev = _gpu_device()
    return native_gpu.unpack_canonical_storage_chunks(
        chunks, bits, source_shape, source_layout, chunk_specs, device=dev).cpu()


def pack_head_channel_chunks(symbols, bits, token_count, num_heads, head_dim, chunk_specs):
    return pack_canonical_storage_chunks(
        symbols, bits, [int(token_count), int(num_heads), int(head_dim)],
        ["token", "head", "head_dim"], chunk_specs)


def unpack_head_channel_chunks(chunks, bits, token_count, num_heads, head_dim, chunk_specs):
    return unpack_canonical_storage_chunks(
        chunks, bits, [int(token_count), int(num_heads), int(head_dim)],
        ["token", "head", "head_dim"], chunk_specs)


def cpu_isa() -> str:
    """Backend tag reported in metrics (the reference reports "cuda")."""
    return "hip"

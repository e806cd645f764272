"""Host-side description of a canonical chunk layout.

Axis naming and validation follow lossless/native_cpu.py:30-130 of the
reference (the aliases and error messages are part of its Python API).  A
CanonicalLayout carries the host metadata arrays every native call needs
(chunk specs, bits, byte offsets), so the hot path never reads metadata back
from the device.
"""
from __future__ import annotations

from dataclasses import dataclass
from functools import cached_property, lru_cache
from typing import Iterable, Sequence

import numpy as np
import torch

_REQUIRED_AXES = ("token", "head", "head_dim")
_AXIS_ALIASES = {
    "token": "token", "tokens": "token", "seq": "token", "sequence": "token",
    "head": "head", "heads": "head", "kv_head": "head", "kv_heads": "head",
    "head_dim": "head_dim", "channel": "head_dim", "channels": "head_dim",
    "dim": "head_dim",
    "layer": "layer", "layers": "layer",
}
STORAGE_LAYOUT = ["layer", "head", "head_dim", "token"]

# The token-major K/V byte view a layer is packed from: a [2, T, H, D] slice of
# the cache with element size e is the uint8 tensor [2T, H, D*e], so each
# (head, byte-channel) token run of a chunk is one byte-plane.
KV_SYMBOL_LAYOUT = ["token", "head", "head_dim"]


def normalize_symbol_layout(layout: Sequence[str]) -> list[str]:
    out: list[str] = []
    for axis in layout:
        key = str(axis).lower()
        if key not in _AXIS_ALIASES:
            raise ValueError(f"Unsupported Origami symbol layout axis {axis!r}")
        out.append(_AXIS_ALIASES[key])
    if len(set(out)) != len(out):
        raise ValueError(f"Origami symbol layout axes must be unique: {layout!r}")
    if any(req not in out for req in _REQUIRED_AXES):
        raise ValueError("Origami symbol layout must include token, head, and head_dim axes")
    extra = set(out) - set(_REQUIRED_AXES) - {"layer"}
    if extra:
        raise ValueError(f"Unsupported Origami symbol layout axes: {sorted(extra)}")
    if len(out) not in (3, 4):
        raise ValueError("Origami symbol layout supports rank 3 or rank 4")
    return out


def canonical_axis_sizes(
    source_shape: Sequence[int], source_layout: Sequence[str]
) -> tuple[int, int, int, list[int], list[str]]:
    shape = [int(d) for d in source_shape]
    layout = normalize_symbol_layout(source_layout)
    if len(shape) != len(layout):
        raise ValueError("origami_symbol_shape rank must match origami_symbol_layout")
    if len(shape) not in (3, 4):
        raise ValueError("origami_symbol_shape supports rank 3 or rank 4")
    if any(d <= 0 for d in shape):
        raise ValueError("origami_symbol_shape dimensions must be positive")
    if "layer" in layout and shape[layout.index("layer")] != 1:
        raise ValueError("per-layer Origami worker requires layer axis size 1")
    return (shape[layout.index("token")], shape[layout.index("head")],
            shape[layout.index("head_dim")], shape, layout)


def axis_positions(source_layout: Sequence[str]) -> list[int]:
    layout = normalize_symbol_layout(source_layout)
    return [layout.index("token"), layout.index("head"), layout.index("head_dim"),
            layout.index("layer") if "layer" in layout else -1]


def specs_array(chunk_specs) -> np.ndarray:
    """[N, 6] int64 host array from a tensor / nested sequence / array."""
    if isinstance(chunk_specs, torch.Tensor):
        arr = chunk_specs.detach().to("cpu", torch.int64).numpy()
    else:
        rows = chunk_specs if isinstance(chunk_specs, np.ndarray) else list(chunk_specs)
        arr = np.asarray(rows, dtype=np.int64) if len(rows) else np.zeros((0, 6), np.int64)
    arr = np.ascontiguousarray(arr, dtype=np.int64)
    if arr.size == 0:
        return np.zeros((0, 6), dtype=np.int64)
    if arr.ndim == 1:
        arr = arr.reshape(1, 6)
    if arr.ndim != 2 or arr.shape[1] != 6:
        raise ValueError("chunk_specs must have shape [N, 6]")
    return arr


def chunk_symbol_counts(specs: np.ndarray) -> np.ndarray:
    return ((specs[:, 1] - specs[:, 0]) * (specs[:, 3] - specs[:, 2])
            * (specs[:, 5] - specs[:, 4]))


@dataclass(frozen=True, eq=False)
class CanonicalLayout:
    """Everything the native calls need to know about one layer's layout."""

    shape: tuple[int, ...]
    layout: tuple[str, ...]
    axes: np.ndarray        # [token, head, head_dim, layer|-1]
    token_count: int
    num_heads: int
    head_dim: int
    specs: np.ndarray       # [N, 6]
    bits: np.ndarray        # [N]
    offsets: np.ndarray     # [N + 1], chunk k holds ceil(n_k * b_k / 8) bytes
    shape_arr: np.ndarray   # shape as int64 array

    @property
    def num_chunks(self) -> int:
        return int(self.specs.shape[0])

    @cached_property
    def torch_meta(self):
        """(offsets, bits, specs) as host int64 tensors sharing the arrays'
        memory, as the extension module's fused entry points take them."""
        import torch

        return (torch.from_numpy(self.offsets), torch.from_numpy(self.bits),
                torch.from_numpy(self.specs))

    @cached_property
    def torch_shape_axes(self):
        """(source shape, axis positions) as host int64 tensors."""
        import torch

        return torch.from_numpy(self.shape_arr), torch.from_numpy(self.axes)

    @cached_property
    def native_args(self) -> tuple[int, int, int, int]:
        """(offsets, bits, specs) host addresses and the chunk count, as the
        C entry points take them; the arrays live as long as the layout."""
        for a in (self.offsets, self.bits, self.specs):
            assert a.flags.c_contiguous and a.dtype == np.int64
        return (self.offsets.ctypes.data, self.bits.ctypes.data, self.specs.ctypes.data,
                int(self.specs.shape[0]))

    @property
    def stream_bytes(self) -> int:
        return int(self.offsets[-1])

    @property
    def symbol_count(self) -> int:
        return int(np.prod(self.shape))

    @property
    def uniform_bits(self) -> int:
        if self.num_chunks == 0:
            return 0
        b = int(self.bits[0])
        return b if bool(np.all(self.bits == b)) else 0

    def chunk_sizes(self) -> list[int]:
        return [int(x) for x in np.diff(self.offsets)]

    @staticmethod
    def make(source_shape: Sequence[int], source_layout: Sequence[str],
             bits: int | Sequence[int], chunk_specs) -> "CanonicalLayout":
        specs = specs_array(chunk_specs)
        if isinstance(bits, (int, np.integer)):
            bits_t: tuple[int, ...] = (int(bits),) * specs.shape[0]
        else:
            bits_t = tuple(int(b) for b in bits)
        if len(bits_t) != specs.shape[0]:
            raise ValueError("bits_per_chunk length must match chunk_specs")
        return _make_cached(tuple(int(d) for d in source_shape),
                            tuple(str(a) for a in source_layout), bits_t,
                            specs.tobytes(), specs.shape[0])


@lru_cache(maxsize=512)
def _make_cached(shape: tuple[int, ...], layout: tuple[str, ...], bits: tuple[int, ...],
                 spec_bytes: bytes, n: int) -> CanonicalLayout:
    T, H, D, shape_l, layout_l = canonical_axis_sizes(shape, layout)
    specs = np.frombuffer(spec_bytes, dtype=np.int64).reshape(n, 6).copy()
    bits_arr = np.asarray(bits, dtype=np.int64).reshape(n)
    if n and (bits_arr.min() < 1 or bits_arr.max() > 8):
        # the reference raises this from its extension (bitpack_layout_cuda.cpp:58-61)
        raise RuntimeError("Origami CUDA bitpack supports only 1..8 bit symbols")
    sizes = (chunk_symbol_counts(specs) * bits_arr + 7) // 8
    offsets = np.zeros(n + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(sizes)
    return CanonicalLayout(
        shape=tuple(shape_l), layout=tuple(layout_l),
        axes=np.asarray(axis_positions(layout_l), dtype=np.int64),
        token_count=T, num_heads=H, head_dim=D,
        specs=specs, bits=bits_arr, offsets=offsets,
        shape_arr=np.asarray(shape_l, dtype=np.int64),
    )


def kv_symbol_layout(tokens: int, num_heads: int, head_bytes: int, bits: int,
                     chunk_specs) -> CanonicalLayout:
    """Layout of one layer's K/V viewed as uint8 [2*tokens, H, head_bytes]."""
    return CanonicalLayout.make([2 * int(tokens), int(num_heads), int(head_bytes)],
                                KV_SYMBOL_LAYOUT, bits, chunk_specs)


def as_chunk_list(chunks: Iterable[torch.Tensor]) -> list[torch.Tensor]:
    return [c.detach().reshape(-1) for c in chunks]

"""Adapter registry (quantization/registry.py:27-47 of the reference).

Registered here: the lossless byte adapters and the CacheGen and KIVI
quantizers, whose restores have fused HIP paths.  KVQuant and TurboQuant are
outside this build."""
from __future__ import annotations

from typing import Any

from origami_amd.quantization.base import QuantizerAdapter
from origami_amd.quantization.cachegen_adapter import CacheGenAdapter
from origami_amd.quantization.kivi_adapter import KiviAdapter
from origami_amd.quantization.raw_tensor import RawBytePlanesAdapter, RawBytesTensorAdapter

_ADAPTERS: dict[str, type[QuantizerAdapter]] = {
    "raw_bytes": RawBytesTensorAdapter,
    "raw": RawBytesTensorAdapter,
    "raw_byte_planes": RawBytePlanesAdapter,
    "byte_planes": RawBytePlanesAdapter,
    "cachegen": CacheGenAdapter,
    "kivi": KiviAdapter,
}


def create_quantizer_adapter(name: str, config: dict[str, Any] | None = None) -> QuantizerAdapter:
    key = str(name).lower()
    if key not in _ADAPTERS:
        raise ValueError(f"Unknown or unsupported Origami quantizer {name!r}; "
                         f"available: {sorted(_ADAPTERS)}")
    return _ADAPTERS[key](config)

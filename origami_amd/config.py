"""Connector configuration (vllm/.../origami/config.py:50-218 of the reference).

Only the fields the layout path reads are modelled; keys keep the reference's
`origami_*` names in kv_connector_extra_config so an existing configuration
is accepted unchanged.  Fields of subsystems outside this build (fused
attention, nvCOMP, QAT tuning, PCIe controller) are parsed and kept, so their
presence is not an error, but have no effect here.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

_DEVICE_POLICIES = {"auto", "cpu", "gpu", "cuda", "hip"}


@dataclass(frozen=True)
class OrigamiConfig:
    quantizer: str = "cachegen"
    quantizer_config: dict[str, Any] = field(default_factory=dict)
    store_uri: str = "memory://origami"
    artifact_format: str = "bundle_v1"
    lossless_cpu_backend: str = "qat"
    allow_zlib_fallback: bool = False
    layout_policy: str = "head_first"
    bitpack: bool = True
    chunk_min_bytes: int = 1 << 20
    chunk_target_bytes: int = 1 << 20
    chunk_max_bytes: int = 1 << 20
    qat_threads: int = 16
    metrics_dir: str = ""
    dequant_device: str = "auto"
    bitunpack_device: str = "auto"
    fused_attention: str = "off"
    # lanes of the layer-wise restore pipeline (one device slot and one stream
    # each); no reference counterpart
    restore_slots: int = 2
    # New (no reference counterpart): the requests of one start_load_kv are
    # restored together, one H2D copy and one batched launch per layer
    batch_restores: bool = True
    read_bandwidth_gbps: float = 0.0
    artifact_ingress_mode: str = "file"
    extra: dict[str, Any] = field(default_factory=dict)

    @classmethod
    def from_extra_config(cls, extra: dict[str, Any] | None) -> "OrigamiConfig":
        extra = dict(extra or {})

        def get(key: str, default: Any) -> Any:
            return extra.get(key, default)

        config = cls(
            quantizer=str(get("origami_quantizer", "cachegen")),
            quantizer_config=dict(get("origami_quantizer_config", {}) or {}),
            store_uri=str(get("origami_store_uri", "memory://origami")),
            artifact_format=str(get("origami_artifact_format", "bundle_v1")),
            lossless_cpu_backend=str(get("origami_lossless_cpu_backend", "qat")),
            allow_zlib_fallback=bool(get("origami_allow_zlib_fallback", False)),
            layout_policy=str(get("origami_layout_policy", "head_first")),
            bitpack=bool(get("origami_bitpack", True)),
            chunk_min_bytes=int(get("origami_chunk_min_bytes", 1 << 20)),
            chunk_target_bytes=int(get("origami_chunk_target_bytes", 1 << 20)),
            chunk_max_bytes=int(get("origami_chunk_max_bytes", 1 << 20)),
            qat_threads=int(get("origami_qat_threads", 16)),
            metrics_dir=str(get("origami_metrics_dir", get("reuse_metrics_dir", ""))),
            dequant_device=str(get("origami_dequant_device", "auto")).lower(),
            bitunpack_device=str(get("origami_bitunpack_device", "auto")).lower(),
            fused_attention=str(get("origami_fused_attention", "off")).lower(),
            restore_slots=int(get("origami_restore_slots", 2)),
            batch_restores=bool(get("origami_batch_restores", True)),
            read_bandwidth_gbps=float(get("origami_read_bandwidth_gbps",
                                          get("reuse_read_bandwidth_gbps", 0.0))),
            artifact_ingress_mode=str(get("origami_artifact_ingress_mode",
                                          get("reuse_artifact_ingress_mode", "file"))).lower(),
            extra=extra,
        )
        config.validate()
        return config

    @classmethod
    def from_vllm_config(cls, vllm_config: Any) -> "OrigamiConfig":
        kv = getattr(vllm_config, "kv_transfer_config", None)
        extra = getattr(kv, "kv_connector_extra_config", None) if kv is not None else None
        return cls.from_extra_config(extra or {})

    def validate(self) -> None:
        if self.chunk_min_bytes <= 0 or self.chunk_target_bytes <= 0 or self.chunk_max_bytes <= 0:
            raise ValueError("Origami chunk sizes must be positive")
        if not (self.chunk_min_bytes <= self.chunk_target_bytes <= self.chunk_max_bytes):
            raise ValueError("origami_chunk_min_bytes <= target <= max is required")
        if self.artifact_format not in {"auto", "bundle_v1", "legacy_pt"}:
            raise ValueError("origami_artifact_format must be one of "
                             "{'auto', 'bundle_v1', 'legacy_pt'}")
        if self.read_bandwidth_gbps < 0:
            raise ValueError("origami_read_bandwidth_gbps must be non-negative")
        if self.artifact_ingress_mode not in {"file", "memory", "native-file"}:
            raise ValueError("origami_artifact_ingress_mode must be one of "
                             "{'file', 'memory', 'native-file'}")
        if self.bitunpack_device not in _DEVICE_POLICIES:
            raise ValueError("origami_bitunpack_device must be auto, cpu, gpu or cuda")
        if self.dequant_device not in _DEVICE_POLICIES:
            raise ValueError("origami_dequant_device must be auto, cpu, gpu or cuda")
        if self.layout_policy not in {"head_first", "layer_token_channel", "baseline"}:
            raise ValueError("origami_layout_policy must be head_first, layer_token_channel "
                             "or baseline")
        if self.restore_slots < 2:
            raise ValueError("origami_restore_slots must be at least 2")

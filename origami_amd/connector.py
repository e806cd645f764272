"""OrigamiConnector: the vLLM KV-connector surface (connector.py:43-257 of the
reference), unchanged in names and semantics for the worker role.

When vLLM is importable the class derives from KVConnectorBase_V1 and
SupportsHMA as the reference does; otherwise a light stand-in base keeps it
usable (the reference's ORIGAMI_LIGHT_IMPORT mode).  The scheduler-role
methods exist for interface compatibility; the scheduler side is outside this
build and raises when used.
"""
from __future__ import annotations

from typing import Any

import torch

from origami_amd.config import OrigamiConfig
from origami_amd.metadata import OrigamiConnectorMetadata
from origami_amd.store import create_origami_store
from origami_amd.worker import OrigamiConnectorWorker

try:  # pragma: no cover - vLLM is not installed in this environment
    from vllm.distributed.kv_transfer.kv_connector.v1 import (
        KVConnectorBase_V1,
        KVConnectorRole,
        SupportsHMA,
    )
    _HAVE_VLLM = True
except Exception:  # noqa: BLE001
    import enum

    _HAVE_VLLM = False

    class KVConnectorRole(enum.Enum):  # noqa: D101
        SCHEDULER = 0
        WORKER = 1

    class KVConnectorBase_V1:  # noqa: D101
        def __init__(self, vllm_config: Any, role: KVConnectorRole,
                     kv_cache_config: Any | None = None):
            self._vllm_config = vllm_config
            self._role = role
            self._kv_cache_config = kv_cache_config
            self._connector_metadata = None

        def bind_connector_metadata(self, connector_metadata: Any) -> None:
            self._connector_metadata = connector_metadata

        def clear_connector_metadata(self) -> None:
            self._connector_metadata = None

    class SupportsHMA:  # noqa: D101
        pass


class OrigamiConnector(KVConnectorBase_V1, SupportsHMA):

    @classmethod
    def get_required_kvcache_layout(cls, vllm_config: Any) -> str | None:
        kv = getattr(vllm_config, "kv_transfer_config", None)
        extra = (getattr(kv, "kv_connector_extra_config", None) if kv is not None else None) or {}
        return "NHD" if str(extra.get("origami_fused_attention", "off")).lower() != "off" else None

    def __init__(self, vllm_config: Any, role: KVConnectorRole,
                 kv_cache_config: Any | None = None, *, config: OrigamiConfig | None = None):
        super().__init__(vllm_config, role, kv_cache_config)
        self.config = config or OrigamiConfig.from_vllm_config(vllm_config)
        self.fused_attention_enabled = False
        if self.config.fused_attention == "required":
            raise ValueError("Origami fused attention is required but is outside this build")
        self.store = create_origami_store(self.config.store_uri,
                                          artifact_format=self.config.artifact_format)
        self.connector_worker: OrigamiConnectorWorker | None = None
        self.connector_scheduler = None
        if role == KVConnectorRole.WORKER:
            self.connector_worker = OrigamiConnectorWorker(self.config, self.store,
                                                           kv_cache_config)

    # ------------------------------------------------------------ worker role

    def register_kv_caches(self, kv_caches: dict[str, torch.Tensor]):
        assert self.connector_worker is not None
        self.connector_worker.register_kv_caches(kv_caches)

    def start_load_kv(self, forward_context: Any, **kwargs: Any) -> None:
        del forward_context, kwargs
        assert self.connector_worker is not None
        assert isinstance(self._connector_metadata, OrigamiConnectorMetadata)
        self.connector_worker.start_load_kv(self._connector_metadata)

    def wait_for_layer_load(self, layer_name: str) -> None:
        assert self.connector_worker is not None
        self.connector_worker.wait_for_layer_load(layer_name)

    def save_kv_layer(self, layer_name: str, kv_layer: torch.Tensor, attn_metadata: Any,
                      **kwargs: Any) -> None:
        del kwargs
        assert self.connector_worker is not None
        self.connector_worker.save_kv_layer(layer_name, kv_layer, attn_metadata)

    def wait_for_save(self):
        assert self.connector_worker is not None
        self.connector_worker.wait_for_save()

    def get_finished(self, finished_req_ids: set[str]) -> tuple[set[str], set[str]]:
        if self.connector_worker is None:
            return set(), set()
        return self.connector_worker.get_finished()

    # -------------------------------------------------------- scheduler role

    def _scheduler_unavailable(self, *_args: Any, **_kwargs: Any):
        raise NotImplementedError("the Origami scheduler side is outside this build")

    get_num_new_matched_tokens = _scheduler_unavailable
    update_state_after_alloc = _scheduler_unavailable
    build_connector_meta = _scheduler_unavailable
    request_finished = _scheduler_unavailable
    request_finished_all_groups = _scheduler_unavailable

    def update_connector_output(self, connector_output: Any) -> None:
        return None

    def get_fused_layer_payloads(self, layer_name: str, request_ids) -> dict:
        return {}

    def get_fused_attention_runtime_config(self) -> dict[str, Any]:
        return {"enabled": False, "mode": self.config.fused_attention}

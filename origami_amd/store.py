"""Artifact store: the in-memory store of the reference (store.py:149-173).

The file-backed bundle_v1 store is not part of this build yet; a
memory:// URI (the reference default) selects this store.
"""
from __future__ import annotations

from threading import Lock

from origami_amd.metadata import OrigamiPayload


class OrigamiStore:
    def put(self, payload: OrigamiPayload) -> None:
        raise NotImplementedError

    def get(self, cache_key: str) -> OrigamiPayload:
        raise NotImplementedError

    def contains(self, cache_key: str) -> bool:
        raise NotImplementedError

    def prepare_for_restore(self, cache_key: str, **_kwargs) -> OrigamiPayload:
        return self.get(cache_key)


class InMemoryOrigamiStore(OrigamiStore):
    _MEMORY: dict[str, OrigamiPayload] = {}
    _MEMORY_LOCK = Lock()

    def __init__(self, namespace: str = "origami"):
        self.namespace = namespace

    def _key(self, cache_key: str) -> str:
        return f"{self.namespace}:{cache_key}"

    def put(self, payload: OrigamiPayload) -> None:
        with self._MEMORY_LOCK:
            self._MEMORY[self._key(payload.cache_key)] = payload

    def get(self, cache_key: str) -> OrigamiPayload:
        with self._MEMORY_LOCK:
            try:
                return self._MEMORY[self._key(cache_key)]
            except KeyError as exc:
                raise KeyError(f"Origami artifact {cache_key!r} is not in the memory store") from exc

    def contains(self, cache_key: str) -> bool:
        with self._MEMORY_LOCK:
            return self._key(cache_key) in self._MEMORY

    def clear(self) -> None:
        with self._MEMORY_LOCK:
            for key in [k for k in self._MEMORY if k.startswith(self.namespace + ":")]:
                del self._MEMORY[key]


def create_origami_store(uri: str, artifact_format: str = "bundle_v1") -> OrigamiStore:
    if uri.startswith("memory://"):
        return InMemoryOrigamiStore(uri[len("memory://"):] or "origami")
    raise ValueError(f"Origami store URI {uri!r} is not supported by this build "
                     "(use memory://<namespace>)")

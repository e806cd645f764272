"""CPU lossless codec (lossless/cpu_qat.py:12-134 of the reference).

Backends: "zlib" (raw DEFLATE, level 1, wbits -15, as cpu_qat.py:64-83) and
"raw" (identity).  Intel QAT ("qat") is outside this build: requesting it
raises unless allow_zlib_fallback is set, which is the reference's behaviour
on a host without QAT devices (cpu_qat.py:41-55).

Chunks are independent, so with threads > 1 the zlib backend compresses and
decompresses them on a thread pool (zlib releases the GIL); the output order
and bytes do not depend on the thread count.
"""
from __future__ import annotations

import zlib
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch


class CpuLosslessCodec:
    def __init__(self, backend: str = "qat", allow_zlib_fallback: bool = False,
                 threads: int = 1, **_unused):
        self.backend = backend
        self.allow_zlib_fallback = allow_zlib_fallback
        self.threads = max(1, int(threads))
        self._pool = ThreadPoolExecutor(max_workers=self.threads) if self.threads > 1 else None
        if backend == "qat":
            if not allow_zlib_fallback:
                raise RuntimeError(
                    "Origami QAT backend is not available. Set "
                    "origami_lossless_cpu_backend='zlib' for tests or enable "
                    "origami_allow_zlib_fallback for development.")
            self.backend = "zlib"
        elif backend not in {"zlib", "raw"}:
            raise ValueError(f"Unsupported Origami CPU lossless backend {backend!r}")

    @staticmethod
    def _cpu_u8(data: torch.Tensor) -> torch.Tensor:
        return data.detach().cpu().to(torch.uint8).reshape(-1).contiguous()

    @staticmethod
    def _zlib_compress(data: torch.Tensor) -> torch.Tensor:
        comp = zlib.compressobj(level=1, wbits=-15, strategy=zlib.Z_DEFAULT_STRATEGY)
        view = memoryview(CpuLosslessCodec._cpu_u8(data).numpy())  # no copy
        out = comp.compress(view) + comp.flush()
        return torch.from_numpy(np.frombuffer(out, dtype=np.uint8).copy())

    @staticmethod
    def _zlib_decompress_into(data: torch.Tensor, out: torch.Tensor) -> None:
        raw = zlib.decompress(memoryview(CpuLosslessCodec._cpu_u8(data).numpy()), wbits=-15)
        if len(raw) != int(out.numel()):
            raise RuntimeError(
                f"Origami CPU lossless decoded {len(raw)} bytes, expected {int(out.numel())}")
        out.numpy()[:] = np.frombuffer(raw, dtype=np.uint8)

    def _map(self, fn, *iterables) -> list:
        """fn over the chunks; on the pool for zlib (plain copies of the raw
        backend are faster on the calling thread than handed to a pool)."""
        items = list(zip(*iterables))
        if self._pool is None or len(items) < 2 or self.backend == "raw":
            return [fn(*a) for a in items]
        return list(self._pool.map(lambda a: fn(*a), items))

    def compress_many(self, chunks) -> list[torch.Tensor]:
        if self.backend == "raw":
            return self._map(self._cpu_u8, chunks)
        return self._map(self._zlib_compress, chunks)

    def decompress_many(self, chunks, output_bytes) -> list[torch.Tensor]:
        if len(chunks) != len(output_bytes):
            raise ValueError("chunks and output_bytes must have the same length")
        outs = [torch.empty((int(n),), dtype=torch.uint8) for n in output_bytes]
        self.decompress_into(chunks, outs)
        return outs

    def decompress_into(self, chunks, outs: list[torch.Tensor]) -> None:
        """Decodes each chunk straight into a caller buffer (e.g. a slice of a
        pinned staging buffer), avoiding an intermediate copy."""
        if len(chunks) != len(outs):
            raise ValueError("chunks and outputs must have the same length")
        self._map(self._raw_into if self.backend == "raw" else self._zlib_decompress_into,
                  chunks, outs)

    @classmethod
    def _raw_into(cls, chunk: torch.Tensor, out: torch.Tensor) -> None:
        flat = cls._cpu_u8(chunk)
        if int(flat.numel()) != int(out.numel()):
            raise RuntimeError(
                "Origami raw backend received "
                f"{int(flat.numel())} bytes, expected {int(out.numel())}")
        out.copy_(flat)

    def compress(self, data: torch.Tensor) -> torch.Tensor:
        return self.compress_many([data])[0]

    def decompress(self, data: torch.Tensor, *, output_bytes: int) -> torch.Tensor:
        return self.decompress_many([data], [int(output_bytes)])[0]

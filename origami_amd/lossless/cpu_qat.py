"""CPU lossless codec (lossless/cpu_qat.py:12-134 of the reference).

Backends: "zlib" (raw DEFLATE, level 1, wbits -15, as cpu_qat.py:64-83) and
"raw" (identity).  Intel QAT ("qat") is outside this build: requesting it
raises unless allow_zlib_fallback is set, which is the reference's behaviour
on a host without QAT devices (cpu_qat.py:41-55).
"""
from __future__ import annotations

import zlib

import torch


class CpuLosslessCodec:
    def __init__(self, backend: str = "qat", allow_zlib_fallback: bool = False, **_unused):
        self.backend = backend
        self.allow_zlib_fallback = allow_zlib_fallback
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
        raw = CpuLosslessCodec._cpu_u8(data).numpy().tobytes()
        out = comp.compress(raw) + comp.flush()
        return torch.frombuffer(bytearray(out), dtype=torch.uint8).clone()

    @staticmethod
    def _zlib_decompress_into(data: torch.Tensor, out: torch.Tensor) -> None:
        raw = zlib.decompress(CpuLosslessCodec._cpu_u8(data).numpy().tobytes(), wbits=-15)
        if len(raw) != int(out.numel()):
            raise RuntimeError(
                f"Origami CPU lossless decoded {len(raw)} bytes, expected {int(out.numel())}")
        out.copy_(torch.frombuffer(bytearray(raw), dtype=torch.uint8))

    def compress_many(self, chunks) -> list[torch.Tensor]:
        if self.backend == "raw":
            return [self._cpu_u8(c) for c in chunks]
        return [self._zlib_compress(c) for c in chunks]

    def decompress_many(self, chunks, output_bytes) -> list[torch.Tensor]:
        if len(chunks) != len(output_bytes):
            raise ValueError("chunks and output_bytes must have the same length")
        outs = [torch.empty((int(n),), dtype=torch.uint8) for n in output_bytes]
        self.decompress_into(chunks, outs)
        return outs

    def decompress_into(self, chunks, outs: list[torch.Tensor]) -> None:
        """Decodes each chunk straight into a caller buffer (e.g. a slice of a
        pinned staging buffer), avoiding an intermediate copy."""
        for chunk, out in zip(chunks, outs):
            if self.backend == "raw":
                flat = self._cpu_u8(chunk)
                if int(flat.numel()) != int(out.numel()):
                    raise RuntimeError(
                        "Origami raw backend received "
                        f"{int(flat.numel())} bytes, expected {int(out.numel())}")
                out.copy_(flat)
            else:
                self._zlib_decompress_into(chunk, out)

    def compress(self, data: torch.Tensor) -> torch.Tensor:
        return self.compress_many([data])[0]

    def decompress(self, data: torch.Tensor, *, output_bytes: int) -> torch.Tensor:
        return self.decompress_many([data], [int(output_bytes)])[0]

"""CacheGen quantizer adapter (quantization/cachegen_adapter.py of the
reference).

CacheGen quantizes each layer's K and V per token with a max-abs affine map
onto `bins` levels whose count depends on the layer (cachegen_adapter.py:
145-182, 246-257).  Payload formats:

* ``cachegen_structured_blob`` (the reference's quantize output,
  cachegen_adapter.py:270-340): one uint8 symbol per value, then the float16
  per-token maxima.
* ``cachegen_bitpacked_blob`` (what the reference's fused restore consumes,
  cachegen_adapter.py:656-819; the reference has no producer for it): the K
  and V symbols packed LSB-first at ``key_bits`` / ``value_bits``
  (bits_for_bins), then the maxima.  This adapter emits it by default
  (``bitpacked`` config key), so that a restore can go through the fused HIP
  unpack + dequantize + paged scatter (native_gpu.
  cachegen_unpack_dequantize_to_kv_cache) in one pass.

Quantize and the unfused dequantize use the reference's torch expressions
(float32 tensor ops, round half to even); they run on whatever device the
input is on.  Bit packing and unpacking run on the GPU (liborigami_layout.so).
"""
from __future__ import annotations

from dataclasses import dataclass
from functools import reduce
from operator import mul
from typing import Any

import torch

from origami_amd.layout import CanonicalLayout
from origami_amd.lossless import native_gpu
from origami_amd.quantization.base import QuantizedKV, QuantizerAdapter

STRUCTURED = "cachegen_structured_blob"
BITPACKED = "cachegen_bitpacked_blob"
_LINEAR_LAYOUT = ("token", "head", "head_dim")


@dataclass(frozen=True)
class CacheGenBins:
    """Layer-dependent bin counts (LMCache's CacheGenConfig fields)."""

    key_first_layers: int
    key_second_layers: int
    key_third_layers: int
    key_first_bins: int
    key_second_bins: int
    key_third_bins: int
    value_first_layers: int
    value_first_bins: int
    value_second_bins: int


def cachegen_bins(model_name: str, quant_level: str) -> CacheGenBins:
    """The bin schedule of cachegen_adapter.py:49-57.  LMCache (whose
    CacheGenConfig the reference tries first, :60-88) is not a dependency of
    this build, and the reference falls back to this table without it."""
    layers = 36 if ("Qwen3-8B" in model_name or "Qwen3_8B" in model_name) else 32
    table = {
        "1": (16, 16, 12, 16, 12),
        "2": (32, 16, 16, 32, 16),
        "3": (32, 32, 32, 32, 32),
    }
    if str(quant_level) not in table:
        raise ValueError(f"Unsupported CacheGen quant_level {quant_level!r}")
    k1, k2, k3, v1, v2 = table[str(quant_level)]
    return CacheGenBins(10, 20, layers, k1, k2, k3, 2, v1, v2)


def layer_index(layer_group: Any | None) -> int:
    """The last run of digits in the layer name (cachegen_adapter.py:99-108)."""
    if layer_group is None:
        return 0
    text = str(layer_group)
    end = len(text)
    while end > 0 and not text[end - 1].isdigit():
        end -= 1
    start = end
    while start > 0 and text[start - 1].isdigit():
        start -= 1
    return int(text[start:end]) if end > start else 0


def bits_for_bins(num_bins: int) -> int:
    """Smallest width holding symbols 0..bins-1, within 1..8
    (cachegen_adapter.py:111-114)."""
    if num_bins <= 1:
        return 1
    return max(1, min(8, int(num_bins - 1).bit_length()))


def dtype_from_metadata(metadata: dict[str, Any]) -> torch.dtype:
    name = str(metadata.get("dtype", "float16")).replace("torch.", "")
    dtype = getattr(torch, name, None)
    if not isinstance(dtype, torch.dtype):
        raise ValueError(f"Unsupported tensor dtype {name!r}")
    return dtype


# ---------------------------------------------------------------------------
# KV layouts (cachegen_adapter.py:184-244; kivi_adapter.py has the same set)
# ---------------------------------------------------------------------------

def canonicalize(kv: torch.Tensor) -> tuple[torch.Tensor, str]:
    """[2, tokens, heads, head_dim] view of a layer's K/V and the name of the
    source layout."""
    t = kv.detach().contiguous()
    s = [int(x) for x in t.shape]
    if t.dim() == 5 and s[0] == 2:
        return t.reshape(2, s[1] * s[2], s[3], s[4]), "kv_blocks_block_heads_dim"
    if t.dim() == 5 and s[1] == 2:
        return (t.permute(1, 0, 2, 3, 4).contiguous().reshape(2, s[0] * s[2], s[3], s[4]),
                "blocks_kv_block_heads_dim")
    if t.dim() == 5 and s[2] == 2:
        return (t.permute(2, 0, 1, 3, 4).contiguous().reshape(2, s[0] * s[1], s[3], s[4]),
                "blocks_block_kv_heads_dim")
    if t.dim() == 4 and s[0] == 2:
        if s[1] <= 128 and s[2] > s[1]:
            return t.permute(0, 2, 1, 3).contiguous(), "kv_heads_tokens_dim"
        return t, "kv_tokens_heads_dim"
    if t.dim() == 4 and s[1] == 2:
        return t.permute(1, 0, 2, 3).contiguous(), "tokens_kv_heads_dim"
    raise ValueError("expected a KV cache layer with a key/value axis; "
                     f"got shape {tuple(kv.shape)}")


def restore_layout(canonical: torch.Tensor, metadata: dict[str, Any]) -> torch.Tensor:
    """Inverse of canonicalize for the layout recorded in `metadata`."""
    shape = [int(d) for d in metadata["shape"]]
    layout = str(metadata["kv_layout"])
    if layout in ("kv_blocks_block_heads_dim", "kv_tokens_heads_dim"):
        return canonical.reshape(shape)
    if layout == "blocks_kv_block_heads_dim":
        return canonical.reshape(2, shape[0], shape[2], shape[3], shape[4]).permute(
            1, 0, 2, 3, 4).contiguous()
    if layout == "blocks_block_kv_heads_dim":
        return canonical.reshape(2, shape[0], shape[1], shape[3], shape[4]).permute(
            1, 2, 0, 3, 4).contiguous()
    if layout == "kv_heads_tokens_dim":
        return canonical.permute(0, 2, 1, 3).contiguous().reshape(shape)
    if layout == "tokens_kv_heads_dim":
        return canonical.permute(1, 0, 2, 3).contiguous().reshape(shape)
    raise ValueError(f"Unsupported KV layout {layout!r}")


def fp16_bytes(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to(torch.float16).contiguous().view(torch.uint8).reshape(-1)


def fp16_view(raw: torch.Tensor, offset: int, numel: int) -> torch.Tensor:
    """float16 values stored at byte `offset` of a uint8 tensor (copied when
    the offset is odd, which a float16 view cannot express)."""
    part = raw.narrow(0, int(offset), int(numel) * 2)
    if int(offset) % 2:
        part = part.clone()
    return part.contiguous().view(torch.float16)


def _linear_layout(count: int, bits: int) -> CanonicalLayout:
    """A [1, 1, count] single-chunk layout: a plain LSB-first bit stream
    (cachegen_adapter.py:117-142)."""
    return CanonicalLayout.make([1, 1, count], _LINEAR_LAYOUT, bits,
                                [[0, 1, 0, count, 0, 1]])


def pack_linear(symbols: torch.Tensor, bits: int) -> torch.Tensor:
    flat = symbols.reshape(-1).to(torch.uint8)
    if flat.numel() == 0:
        return torch.empty((0,), dtype=torch.uint8, device=flat.device)
    dev = flat.device if flat.is_cuda else torch.device("cuda")
    return native_gpu.pack_layout(flat.to(dev).contiguous(), _linear_layout(flat.numel(), bits))


def unpack_linear(raw: torch.Tensor, bits: int, count: int) -> torch.Tensor:
    if count == 0:
        return torch.empty((0,), dtype=torch.uint8, device=raw.device)
    layout = _linear_layout(count, bits)
    dev = raw.device if raw.is_cuda else torch.device("cuda")
    flat = raw.reshape(-1).to(dev, torch.uint8)
    if flat.numel() < layout.stream_bytes:
        raise RuntimeError("CacheGen symbol stream is shorter than its symbol count")
    return native_gpu.unpack_layout(flat[: layout.stream_bytes].contiguous(), layout)


def dequantize_into_cache(adapter, raw: torch.Tensor, metadata: dict[str, Any],
                          dst_cache: torch.Tensor, block_ids) -> torch.cuda.Event:
    """Shared by the CacheGen and KIVI adapters: the fused restore when it
    applies, else the unfused dequantize plus a block scatter.  The scatter is
    copy_kv_to_hbm, which handles both cache layouts and zero-pads a partial
    last block; the reference assigns dst_cache[block_ids] instead, which is
    right for [num_blocks, 2, ...] caches only (cachegen_adapter.py:913-917)."""
    from origami_amd.benchmark_utils import copy_kv_to_hbm

    tokens = int(metadata["token_count"])
    if adapter.can_dequantize_to_cache(metadata, dst_cache, block_ids, tokens=tokens):
        ids = torch.as_tensor(list(block_ids), dtype=torch.int64).to(dst_cache.device)
        adapter.dequantize_to_cache(raw.to(dst_cache.device), metadata, dst_cache, ids, tokens)
        event = torch.cuda.Event()
        event.record(torch.cuda.current_stream(dst_cache.device))
        return event
    dense = adapter._dequantize_dense(raw.to(dst_cache.device), metadata)
    _, event = copy_kv_to_hbm(kv_cache=dst_cache, block_ids=list(block_ids),
                              value=dense.to(dst_cache.dtype), request_id="dequantize",
                              cache_key="", system="origami", layer_name="",
                              synchronize=False, return_event=True)
    return event


class CacheGenAdapter(QuantizerAdapter):
    """CacheGen per-layer max-abs quantizer (cachegen_adapter.py:145-938)."""

    quantizer_id = "cachegen"

    def __init__(self, config: dict[str, Any] | None = None):
        super().__init__(config)
        self.model_name = str(self.config.get("model_name", "/data/llm/Mistral-7B-Instruct-v0.2"))
        self.quant_level = str(self.config.get("quant_level", "2"))
        self.dequant_device = str(self.config.get("dequant_device", "auto")).lower()
        self.bitpacked = bool(self.config.get("bitpacked", True))
        self.bins = cachegen_bins(self.model_name, self.quant_level)
        if self.dequant_device not in {"auto", "cpu", "gpu", "cuda"}:
            raise ValueError("CacheGenAdapter dequant_device must be one of "
                             "{'auto', 'cpu', 'gpu', 'cuda'}")

    def key_bins(self, layer: int) -> int:
        b = self.bins
        if layer < b.key_first_layers:
            return b.key_first_bins
        if layer < b.key_second_layers:
            return b.key_second_bins
        return b.key_third_bins

    def value_bins(self, layer: int) -> int:
        b = self.bins
        return b.value_first_bins if layer < b.value_first_layers else b.value_second_bins

    # -- quantize ------------------------------------------------------------

    @staticmethod
    def quantize_plane(plane: torch.Tensor, bins: int) -> tuple[torch.Tensor, torch.Tensor]:
        """[tokens, ...] -> uint8 symbols [tokens, C] and float16 maxima
        [tokens, 1] (cachegen_adapter.py:246-257)."""
        tokens = int(plane.shape[0])
        x = plane.reshape(tokens, -1).to(torch.float32)
        max_abs = torch.amax(torch.abs(x), dim=-1, keepdim=True).clamp_min(1e-6)
        center = bins // 2 - 1
        q = torch.round(x * (center / max_abs) + center).clamp(0, center * 2).to(torch.uint8)
        return q, max_abs.to(torch.float16)

    def quantize(self, kv: torch.Tensor, *, request: Any | None = None,
                 layer_group: Any | None = None, stream: Any | None = None) -> QuantizedKV:
        del request, stream
        canonical, layout = canonicalize(kv)
        layer = layer_index(layer_group)
        kbins, vbins = self.key_bins(layer), self.value_bins(layer)
        kbits, vbits = bits_for_bins(kbins), bits_for_bins(vbins)
        key_q, key_max = self.quantize_plane(canonical[0], kbins)
        value_q, value_max = self.quantize_plane(canonical[1], vbins)
        tokens, heads, head_dim = (int(x) for x in canonical.shape[1:])
        meta: dict[str, Any] = {
            "format": BITPACKED if self.bitpacked else STRUCTURED,
            "version": 2,
            "model_name": self.model_name,
            "quant_level": self.quant_level,
            "layer_index": layer,
            "key_bins": kbins,
            "value_bins": vbins,
            "key_bits": kbits,
            "value_bits": vbits,
            "dtype": str(kv.dtype).replace("torch.", ""),
            "shape": [int(d) for d in kv.shape],
            "kv_layout": layout,
            "token_count": tokens,
            "num_heads": heads,
            "head_dim": head_dim,
            "channel_count": heads * head_dim,
            "key_q_numel": int(key_q.numel()),
            "value_q_numel": int(value_q.numel()),
            "key_max_numel": int(key_max.numel()),
            "value_max_numel": int(value_max.numel()),
        }
        if self.bitpacked:
            streams = [pack_linear(key_q, kbits), pack_linear(value_q, vbits)]
            names = ["key_stream", "value_stream"]
        else:
            streams = [key_q.reshape(-1), value_q.reshape(-1)]
            names = ["key_q", "value_q"]
        parts, cursor = [], 0
        dev = streams[0].device
        for name, part in zip(names + ["key_max", "value_max"],
                              streams + [fp16_bytes(key_max).to(dev), fp16_bytes(value_max).to(dev)]):
            if name.endswith("_max") and cursor % 2:     # float16 views need even offsets
                parts.append(torch.zeros((1,), dtype=torch.uint8, device=dev))
                cursor += 1
            meta[f"{name}_offset"] = cursor
            if name.endswith("_stream"):
                meta[f"{name}_bytes"] = int(part.numel())
            parts.append(part.reshape(-1).to(torch.uint8))
            cursor += int(part.numel())
        symbols = torch.cat(parts).contiguous()
        meta.update({
            "symbol_byte_count": int(symbols.numel()),
            "origami_bits": 8,
            "origami_symbol_shape": [1, 1, int(symbols.numel())],
            "origami_symbol_layout": list(_LINEAR_LAYOUT),
            "origami_data_layout_policy": "layer>head>head_dim>token",
        })
        return QuantizedKV(symbols=symbols, metadata=meta)

    # -- dequantize ------------------------------------------------------------

    @staticmethod
    def dequantize_plane(q: torch.Tensor, max_abs: torch.Tensor, bins: int) -> torch.Tensor:
        """cachegen_adapter.py:364-370."""
        center = bins // 2 - 1
        return (q.to(torch.float32) - center) / center * max_abs

    def _use_gpu(self) -> bool:
        if self.dequant_device == "cpu":
            return False
        if not torch.cuda.is_available():
            if self.dequant_device in {"gpu", "cuda"}:
                raise RuntimeError("CacheGenAdapter GPU dequant requested but no GPU is visible")
            return False
        return True

    def can_dequantize_to_cache(self, metadata: dict[str, Any], dst_cache: torch.Tensor,
                                block_ids, *, tokens: int | None = None) -> bool:
        """When the fused restore applies (cachegen_adapter.py:656-700): a
        bit-packed payload, a float16/bfloat16 rank-5 GPU cache of matching
        heads, and whole blocks (the fused kernel leaves tail tokens as they
        are, so partial blocks take the zero-padding unfused path)."""
        if str(metadata.get("format")) != BITPACKED or not self._use_gpu():
            return False
        if not dst_cache.is_cuda or dst_cache.dtype not in (torch.float16, torch.bfloat16):
            return False
        if dst_cache.dim() != 5 or len(block_ids) == 0:
            return False
        if int(dst_cache.shape[1]) != 2 and int(dst_cache.shape[0]) != 2:
            return False
        bs, heads, head_dim = (int(x) for x in dst_cache.shape[2:])
        restore_tokens = int(tokens if tokens is not None else metadata["token_count"])
        if restore_tokens <= 0 or restore_tokens % bs != 0:
            return False
        if restore_tokens > len(block_ids) * bs:
            return False
        return heads == int(metadata["num_heads"]) and head_dim == int(metadata["head_dim"])

    def dequantize_to_cache(self, raw: torch.Tensor, metadata: dict[str, Any],
                            dst_cache: torch.Tensor, block_ids: torch.Tensor,
                            tokens: int) -> None:
        """Fused restore of a bit-packed payload already on the GPU, enqueued
        on the current stream (cachegen_adapter.py:702-819)."""
        tokens_all = int(metadata["token_count"])
        native_gpu.cachegen_unpack_dequantize_to_kv_cache(
            raw, key_offset=int(metadata["key_stream_offset"]),
            key_bytes=int(metadata["key_stream_bytes"]),
            value_offset=int(metadata["value_stream_offset"]),
            value_bytes=int(metadata["value_stream_bytes"]),
            key_bits=int(metadata["key_bits"]), value_bits=int(metadata["value_bits"]),
            key_bins=int(metadata["key_bins"]), value_bins=int(metadata["value_bins"]),
            max_key=fp16_view(raw, metadata["key_max_offset"], tokens_all),
            max_value=fp16_view(raw, metadata["value_max_offset"], tokens_all),
            kv_cache=dst_cache, block_ids=block_ids, tokens=int(tokens),
            heads=int(metadata["num_heads"]), head_dim=int(metadata["head_dim"]))

    def _dequantize_dense(self, raw: torch.Tensor, metadata: dict[str, Any]) -> torch.Tensor:
        fmt = str(metadata.get("format"))
        tokens = int(metadata["token_count"])
        C = int(metadata["channel_count"])
        heads, head_dim = int(metadata["num_heads"]), int(metadata["head_dim"])
        if fmt == BITPACKED:
            key_q = unpack_linear(raw.narrow(0, int(metadata["key_stream_offset"]),
                                             int(metadata["key_stream_bytes"])),
                                  int(metadata["key_bits"]), int(metadata["key_q_numel"]))
            value_q = unpack_linear(raw.narrow(0, int(metadata["value_stream_offset"]),
                                               int(metadata["value_stream_bytes"])),
                                    int(metadata["value_bits"]), int(metadata["value_q_numel"]))
            key_q, value_q = key_q.to(raw.device), value_q.to(raw.device)
        else:
            key_q = raw.narrow(0, int(metadata["key_q_offset"]), int(metadata["key_q_numel"]))
            value_q = raw.narrow(0, int(metadata["value_q_offset"]),
                                 int(metadata["value_q_numel"]))
        key_max = fp16_view(raw, metadata["key_max_offset"], metadata["key_max_numel"])
        value_max = fp16_view(raw, metadata["value_max_offset"], metadata["value_max_numel"])
        key = self.dequantize_plane(key_q.reshape(tokens, C), key_max.float().reshape(-1, 1),
                                    int(metadata["key_bins"]))
        value = self.dequantize_plane(value_q.reshape(tokens, C),
                                      value_max.float().reshape(-1, 1),
                                      int(metadata["value_bins"]))
        canonical = torch.stack([key.reshape(tokens, heads, head_dim),
                                 value.reshape(tokens, heads, head_dim)], dim=0)
        return restore_layout(canonical.to(dtype_from_metadata(metadata)), metadata)

    def dequantize(self, symbols: torch.Tensor, metadata: dict[str, Any], *,
                   dst_cache: torch.Tensor | None = None, block_ids=None,
                   stream: Any | None = None) -> torch.Tensor | Any:
        del stream
        fmt = str(metadata.get("format"))
        if fmt not in {STRUCTURED, BITPACKED, "cachegen_quantized_blob"}:
            raise ValueError("CacheGenAdapter can only dequantize CacheGen Origami payloads")
        raw = symbols.detach().reshape(-1).to(torch.uint8)
        expected = int(metadata.get("symbol_byte_count", raw.numel()))
        if int(raw.numel()) != expected:
            raise RuntimeError(f"CacheGen quantized payload size mismatch: got "
                               f"{int(raw.numel())}, expected {expected}")
        if dst_cache is not None and block_ids is not None:
            return dequantize_into_cache(self, raw, metadata, dst_cache, block_ids)
        device = torch.device("cuda") if self._use_gpu() or fmt == BITPACKED else raw.device
        tensor = self._dequantize_dense(raw.to(device), metadata)
        if reduce(mul, tensor.shape, 1) != reduce(mul, [int(d) for d in metadata["shape"]], 1):
            raise RuntimeError("CacheGen dequantized tensor shape mismatch")
        return tensor

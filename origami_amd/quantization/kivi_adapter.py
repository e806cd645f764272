"""KIVI quantizer adapter (quantization/kivi_adapter.py of the reference).

KIVI quantizes keys per channel with groups of `group_size` tokens and values
per token with groups of `group_size` channels, keeping the first
`sink_tokens` tokens in float16 (kivi_adapter.py:125-450).  The payload
(``kivi_structured_blob``) is one byte blob: the key stream (symbol order
head_dim > layer > head > token), the value stream (head > layer > head_dim >
token), then float16 key scale / zero ([key_groups, C]), value scale / zero
([body, value_groups]) and key / value sink values ([sink, C]), each at an
even offset.  Streams use KIVI's packers: 2 and 4 bits LSB-first, 8 bits as
bytes, 3 bits one symbol per nibble (kivi_adapter.py:28-54).

Restore paths:
* fused (can_dequantize_to_cache): native_gpu.kivi_dequantize_to_kv_cache
  reads the blob on the GPU and writes the paged cache in one pass, with the
  reference kernel's arithmetic (one fused multiply-add per value, rounded
  once to the cache dtype, bitpack_layout_cuda.cu:578-683);
* unfused (dequantize without a cache): the reference's torch expressions
  (kivi_adapter.py:453-531: separate multiply and add in float32, rounded to
  float16, then cast to the payload dtype).
"""
from __future__ import annotations

from typing import Any

import torch

from origami_amd.lossless import native_gpu
from origami_amd.quantization.base import QuantizedKV, QuantizerAdapter
from origami_amd.quantization.cachegen_adapter import (
    canonicalize,
    dequantize_into_cache,
    dtype_from_metadata,
    fp16_bytes,
    fp16_view,
    restore_layout,
)

FORMAT = "kivi_structured_blob"
KEY_ORDER = ("head_dim", "layer", "head", "token")
VALUE_ORDER = ("head", "layer", "head_dim", "token")
_AXES = ("layer", "token", "head", "head_dim")


def pack_lowbit(values: torch.Tensor, bits: int) -> torch.Tensor:
    """kivi_adapter.py:28-54, on the tensor's device."""
    v = values.reshape(-1).to(torch.uint8)
    if v.numel() == 0:
        return torch.empty((0,), dtype=torch.uint8, device=v.device)
    if bits == 8:
        return v.clone()
    if bits in (3, 4):
        if v.numel() % 2:
            v = torch.cat([v, v.new_zeros(1)])
        pairs = v.reshape(-1, 2)
        m = 0x07 if bits == 3 else 0x0F
        return ((pairs[:, 0] & m) | ((pairs[:, 1] & m) << 4)).contiguous()
    if bits == 2:
        pad = (-v.numel()) % 4
        if pad:
            v = torch.cat([v, v.new_zeros(pad)])
        g = v.reshape(-1, 4) & 0x03
        return (g[:, 0] | (g[:, 1] << 2) | (g[:, 2] << 4) | (g[:, 3] << 6)).contiguous()
    raise ValueError("KIVI adapter supports only 2, 3, 4, or 8 bit packing")


def unpack_lowbit(data: torch.Tensor, bits: int, count: int) -> torch.Tensor:
    """kivi_adapter.py:57-94, on the tensor's device."""
    src = data.reshape(-1).to(torch.uint8)
    if count == 0:
        return torch.empty((0,), dtype=torch.uint8, device=src.device)
    if bits == 8:
        return src[:count].clone()
    per = {2: 4, 3: 2, 4: 2}.get(bits)
    if per is None:
        raise ValueError("KIVI adapter supports only 2, 3, 4, or 8 bit packing")
    width = 8 // per
    m = 0x07 if bits == 3 else (1 << width) - 1
    out = torch.stack([(src >> (width * k)) & m for k in range(per)], dim=1).reshape(-1)
    return out[:count].contiguous()


def pack_ordered(q: torch.Tensor, order: tuple[str, ...], bits: int) -> torch.Tensor:
    """q: [1, body, heads, head_dim] symbols -> packed stream in `order`."""
    return pack_lowbit(q.permute(*[_AXES.index(a) for a in order]).contiguous(), bits)


def unpack_ordered(data: torch.Tensor, shape: tuple[int, int, int, int], order: tuple[str, ...],
                   bits: int) -> torch.Tensor:
    dims = [_AXES.index(a) for a in order]
    count = shape[0] * shape[1] * shape[2] * shape[3]
    vals = unpack_lowbit(data, bits, count).reshape([shape[d] for d in dims])
    inverse = [0] * 4
    for i, d in enumerate(dims):
        inverse[d] = i
    return vals.permute(*inverse).contiguous()


class KiviAdapter(QuantizerAdapter):
    """KIVI grouped asymmetric quantizer (kivi_adapter.py:125-733)."""

    quantizer_id = "kivi"

    def __init__(self, config: dict[str, Any] | None = None):
        super().__init__(config)
        self.bits = int(self.config.get("bits", self.config.get("kivi_bits", 2)))
        self.group_size = int(self.config.get("group_size",
                                              self.config.get("kivi_group_size", 64)))
        self.sink_tokens = int(self.config.get("sink_tokens",
                                               self.config.get("kivi_sink_tokens", 128)))
        self.dequant_device = str(self.config.get("dequant_device", "auto")).lower()
        if self.bits not in {2, 3, 4, 8}:
            raise ValueError("KiviAdapter bits must be one of {2, 3, 4, 8}")
        if self.group_size <= 0:
            raise ValueError("KiviAdapter group_size must be positive")
        if self.sink_tokens < 0:
            raise ValueError("KiviAdapter sink_tokens must be non-negative")
        if self.dequant_device not in {"auto", "cpu", "gpu", "cuda"}:
            raise ValueError("KiviAdapter dequant_device must be one of "
                             "{'auto', 'cpu', 'gpu', 'cuda'}")

    # -- quantize ------------------------------------------------------------

    @staticmethod
    def quantize_key_per_channel(m: torch.Tensor, group: int, bits: int):
        """[rows, cols] float32 -> symbols, scale, zero over token groups
        (kivi_adapter.py:229-257)."""
        rows, cols = int(m.shape[0]), int(m.shape[1])
        groups = (rows + group - 1) // group
        if rows == 0:
            return (m.new_empty((0, cols), dtype=torch.uint8),
                    m.new_empty((0, cols), dtype=torch.float16),
                    m.new_empty((0, cols), dtype=torch.float16))
        pad = groups * group - rows
        padded = m if pad == 0 else torch.cat([m, m[-1:].expand(pad, cols)], dim=0)
        g = padded.reshape(groups, group, cols)
        zero = torch.amin(g, dim=1)
        levels = float((1 << bits) - 1)
        scale = torch.clamp((torch.amax(g, dim=1) - zero) / levels,
                            min=torch.finfo(torch.float32).tiny)
        q = torch.round((g - zero[:, None, :]) / scale[:, None, :]).clamp(0, levels)
        return (q.to(torch.uint8).reshape(groups * group, cols)[:rows].contiguous(),
                scale.to(torch.float16).contiguous(), zero.to(torch.float16).contiguous())

    @staticmethod
    def quantize_value_per_token(m: torch.Tensor, group: int, bits: int):
        """[rows, cols] float32 -> symbols, scale, zero over channel groups
        (kivi_adapter.py:259-288)."""
        rows, cols = int(m.shape[0]), int(m.shape[1])
        groups = (cols + group - 1) // group
        if rows == 0:
            return (m.new_empty((0, cols), dtype=torch.uint8),
                    m.new_empty((0, groups), dtype=torch.float16),
                    m.new_empty((0, groups), dtype=torch.float16))
        pad = groups * group - cols
        padded = m if pad == 0 else torch.cat([m, m[:, -1:].expand(rows, pad)], dim=1)
        g = padded.reshape(rows, groups, group)
        zero = torch.amin(g, dim=2)
        levels = float((1 << bits) - 1)
        scale = torch.clamp((torch.amax(g, dim=2) - zero) / levels,
                            min=torch.finfo(torch.float32).tiny)
        q = torch.round((g - zero[:, :, None]) / scale[:, :, None]).clamp(0, levels)
        return (q.to(torch.uint8).reshape(rows, groups * group)[:, :cols].contiguous(),
                scale.to(torch.float16).contiguous(), zero.to(torch.float16).contiguous())

    def quantize(self, kv: torch.Tensor, *, request: Any | None = None,
                 layer_group: Any | None = None, stream: Any | None = None) -> QuantizedKV:
        del request, layer_group, stream
        canonical, layout = canonicalize(kv)
        c16 = canonical.to(torch.float16).contiguous()
        tokens, heads, head_dim = (int(x) for x in c16.shape[1:])
        sink = min(self.sink_tokens, tokens)
        body = tokens - sink
        cols = heads * head_dim
        key_q, key_scale, key_zero = self.quantize_key_per_channel(
            c16[0, sink:].reshape(body, cols).float(), self.group_size, self.bits)
        value_q, value_scale, value_zero = self.quantize_value_per_token(
            c16[1, sink:].reshape(body, cols).float(), self.group_size, self.bits)
        data_shape = (1, body, heads, head_dim)
        key_stream = pack_ordered(key_q.reshape(data_shape), KEY_ORDER, self.bits)
        value_stream = pack_ordered(value_q.reshape(data_shape), VALUE_ORDER, self.bits)
        parts, offsets, cursor = [], {}, 0
        dev = key_stream.device
        named = [("key_stream", key_stream, 1), ("value_stream", value_stream, 1),
                 ("key_scale", fp16_bytes(key_scale), 2), ("key_zero", fp16_bytes(key_zero), 2),
                 ("value_scale", fp16_bytes(value_scale), 2),
                 ("value_zero", fp16_bytes(value_zero), 2),
                 ("key_sink", fp16_bytes(c16[0, :sink]), 2),
                 ("value_sink", fp16_bytes(c16[1, :sink]), 2)]
        for name, data, align in named:
            pad = (-cursor) % align
            if pad:
                parts.append(torch.zeros((pad,), dtype=torch.uint8, device=dev))
                cursor += pad
            offsets[name] = cursor
            parts.append(data.reshape(-1).to(dev, torch.uint8))
            cursor += int(data.numel())
        symbols = torch.cat(parts).contiguous()
        meta: dict[str, Any] = {
            "format": FORMAT,
            "version": 1,
            "bits": self.bits,
            "group_size": self.group_size,
            "sink_tokens": sink,
            "body_tokens": body,
            "token_count": tokens,
            "num_heads": heads,
            "head_dim": head_dim,
            "channel_count": cols,
            "key_groups": (body + self.group_size - 1) // self.group_size,
            "value_groups": (cols + self.group_size - 1) // self.group_size,
            "data_shape": list(data_shape),
            "key_order": list(KEY_ORDER),
            "value_order": list(VALUE_ORDER),
            "dtype": str(kv.dtype).replace("torch.", ""),
            "shape": [int(d) for d in kv.shape],
            "kv_layout": layout,
            "symbol_byte_count": int(symbols.numel()),
            "origami_bits": 8,
            "origami_symbol_shape": [1, 1, int(symbols.numel())],
            "origami_symbol_layout": ["token", "head", "head_dim"],
        }
        for name, off in offsets.items():
            meta[f"{name}_offset"] = int(off)
        meta.update({
            "key_stream_bytes": int(key_stream.numel()),
            "value_stream_bytes": int(value_stream.numel()),
            "key_scale_numel": int(key_scale.numel()),
            "key_zero_numel": int(key_zero.numel()),
            "value_scale_numel": int(value_scale.numel()),
            "value_zero_numel": int(value_zero.numel()),
            "key_sink_numel": int(sink * cols),
            "value_sink_numel": int(sink * cols),
        })
        return QuantizedKV(symbols=symbols, metadata=meta)

    # -- dequantize ------------------------------------------------------------

    def _use_gpu(self) -> bool:
        if self.dequant_device == "cpu":
            return False
        if not torch.cuda.is_available():
            if self.dequant_device in {"gpu", "cuda"}:
                raise RuntimeError("KiviAdapter GPU dequant requested but no GPU is visible")
            return False
        return True

    def can_dequantize_to_cache(self, metadata: dict[str, Any], dst_cache: torch.Tensor,
                                block_ids, *, tokens: int | None = None) -> bool:
        """kivi_adapter.py:537-571: a KIVI payload restored whole, into a
        float16/bfloat16 rank-5 GPU cache of matching heads, in whole blocks."""
        if str(metadata.get("format")) != FORMAT or not self._use_gpu():
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
        return (restore_tokens == int(metadata["token_count"])
                and heads == int(metadata["num_heads"]) and head_dim == int(metadata["head_dim"]))

    def dequantize_to_cache(self, raw: torch.Tensor, metadata: dict[str, Any],
                            dst_cache: torch.Tensor, block_ids: torch.Tensor,
                            tokens: int) -> None:
        """Fused restore of a payload already on the GPU, enqueued on the
        current stream (kivi_adapter.py:573-683)."""
        def meta(name: str) -> torch.Tensor:
            return fp16_view(raw, metadata[f"{name}_offset"], metadata[f"{name}_numel"])

        native_gpu.kivi_dequantize_to_kv_cache(
            raw, key_offset=int(metadata["key_stream_offset"]),
            key_bytes=int(metadata["key_stream_bytes"]),
            value_offset=int(metadata["value_stream_offset"]),
            value_bytes=int(metadata["value_stream_bytes"]), bits=int(metadata["bits"]),
            group_size=int(metadata["group_size"]), sink_tokens=int(metadata["sink_tokens"]),
            key_scale=meta("key_scale"), key_zero=meta("key_zero"),
            value_scale=meta("value_scale"), value_zero=meta("value_zero"),
            key_sink=meta("key_sink"), value_sink=meta("value_sink"), kv_cache=dst_cache,
            block_ids=block_ids, tokens=int(tokens), heads=int(metadata["num_heads"]),
            head_dim=int(metadata["head_dim"]), symbol_packing="kivi")

    def _dequantize_dense(self, raw: torch.Tensor, metadata: dict[str, Any]) -> torch.Tensor:
        """kivi_adapter.py:453-531 (unfused arithmetic, float16 intermediate)."""
        tokens, body = int(metadata["token_count"]), int(metadata["body_tokens"])
        sink = int(metadata["sink_tokens"])
        heads, head_dim = int(metadata["num_heads"]), int(metadata["head_dim"])
        cols = heads * head_dim
        bits, group = int(metadata["bits"]), int(metadata["group_size"])
        shape = tuple(int(d) for d in metadata["data_shape"])
        key_q = unpack_ordered(raw.narrow(0, int(metadata["key_stream_offset"]),
                                          int(metadata["key_stream_bytes"])),
                               shape, tuple(metadata["key_order"]), bits).reshape(body, cols)
        value_q = unpack_ordered(raw.narrow(0, int(metadata["value_stream_offset"]),
                                            int(metadata["value_stream_bytes"])),
                                 shape, tuple(metadata["value_order"]), bits).reshape(body, cols)

        def meta(name: str) -> torch.Tensor:
            return fp16_view(raw, metadata[f"{name}_offset"], metadata[f"{name}_numel"])

        key_scale = meta("key_scale").reshape(int(metadata["key_groups"]), cols).float()
        key_zero = meta("key_zero").reshape(int(metadata["key_groups"]), cols).float()
        value_scale = meta("value_scale").reshape(body, int(metadata["value_groups"])).float()
        value_zero = meta("value_zero").reshape(body, int(metadata["value_groups"])).float()
        key_sink = meta("key_sink").reshape(sink, heads, head_dim)
        value_sink = meta("value_sink").reshape(sink, heads, head_dim)
        if body > 0:
            rows = torch.arange(body, device=raw.device) // group
            cols_g = torch.arange(cols, device=raw.device) // group
            key_body = key_q.float() * key_scale[rows, :] + key_zero[rows, :]
            value_body = value_q.float() * value_scale[:, cols_g] + value_zero[:, cols_g]
            key = torch.cat([key_sink, key_body.reshape(body, heads, head_dim).half()], dim=0)
            value = torch.cat([value_sink, value_body.reshape(body, heads, head_dim).half()],
                              dim=0)
        else:
            key, value = key_sink, value_sink
        if int(key.shape[0]) != tokens or int(value.shape[0]) != tokens:
            raise RuntimeError("KIVI dequantized token count mismatch")
        canonical = torch.stack([key, value], dim=0).to(dtype_from_metadata(metadata))
        return restore_layout(canonical, metadata)

    def dequantize(self, symbols: torch.Tensor, metadata: dict[str, Any], *,
                   dst_cache: torch.Tensor | None = None, block_ids=None,
                   stream: Any | None = None) -> torch.Tensor | Any:
        del stream
        if str(metadata.get("format")) != FORMAT:
            raise ValueError("KiviAdapter can only dequantize KIVI Origami payloads")
        raw = symbols.detach().reshape(-1).to(torch.uint8)
        expected = int(metadata["symbol_byte_count"])
        if int(raw.numel()) != expected:
            raise RuntimeError(f"KIVI payload size mismatch: got {int(raw.numel())}, "
                               f"expected {expected}")
        if dst_cache is not None and block_ids is not None:
            return dequantize_into_cache(self, raw, metadata, dst_cache, block_ids)
        device = torch.device("cuda") if self._use_gpu() else raw.device
        return self._dequantize_dense(raw.to(device), metadata)

from origami_amd.quantization.base import QuantizedKV, QuantizerAdapter
from origami_amd.quantization.registry import create_quantizer_adapter

__all__ = ["QuantizedKV", "QuantizerAdapter", "create_quantizer_adapter"]
